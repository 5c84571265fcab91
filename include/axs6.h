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
 *     element at flat index i from a keyed hash of the counter offset + i
 *     (key = splitmix64 finaliser of seed; a 32-bit multiply-xorshift hash
 *     per element; top 24 bits), so a (seed, offset) pair reproduces a draw
 *     exactly.  The stochastic entry points also take `seed_dev`, a device
 *     pointer (may be NULL) whose uint64 value, read when the kernel runs, is
 *     added to `seed`: a call recorded in a HIP graph then draws fresh values
 *     on every replay when the caller advances that counter.
 *
 * Python binding: axs-6_amd/axs/_lib.py (ctypes).  The reference entry
 * point each call replaces is cited on its declaration.
 */
#ifndef AXS6_H
#define AXS6_H

#include <stddef.h>
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
                           uint64_t offset, const uint64_t* seed_dev, void* stream);

/* NF5 quantize to the AXSTensor fields, optionally also writing FQ(x):
 *   exponents  u8 [rows, nblk]            (nblk = ceil(cols / block_size))
 *   codes      u8 [rows, nblk*block_size] 5-bit NF5 magnitude codes
 *   signs      u8 [rows, nblk*block_size] 1 where x < 0 (may be NULL)
 *   fq         same dtype as x [rows, cols], fused_fake_quantize of x (may be NULL)
 * Replaces: quantize_unified (axs/unified/quantize_unified.py:211). */
int axs6_nf5_quantize(const void* x, int32_t dtype, int64_t rows, int64_t cols,
                      int32_t block_size, int32_t stochastic, uint64_t seed, uint64_t offset,
                      uint8_t* exponents, uint8_t* codes, uint8_t* signs, void* fq,
                      const uint64_t* seed_dev, void* stream);

/* Inverse of axs6_nf5_quantize: y[rows, cols] f32 = +-codebook[code] * 2^(e-127).
 * Replaces: dequantize_unified (axs/unified/quantize_unified.py:285). */
int axs6_nf5_dequantize(const uint8_t* exponents, const uint8_t* codes, const uint8_t* signs,
                        float* y, int64_t rows, int64_t cols, int32_t block_size, void* stream);

/* ---- NF5 wire format ---------------------------------------------------------
 * The 6.25-bit encoding of a gradient: per block of block_size values (blocks
 * in row-major order, the last block of a row zero-padded), one record of
 * 1 + block_size*3/4 bytes: byte 0 the shared exponent (quantize's rule),
 * then 6-bit codes q = (sign << 5) | code, four per three bytes, low bits
 * first (b0 = q0 | q1<<6, b1 = q1>>2 | q2<<4, b2 = q2>>4 | q3<<2).  A 32-value
 * block takes 25 bytes.  Codes use nearest rounding.
 */

/* Bytes of the wire buffer for a rows x cols tensor (-1 on bad arguments). */
int64_t axs6_nf5_wire_bytes(int64_t rows, int64_t cols, int32_t block_size);

/* Quantize x [rows, cols] (`dtype`) straight into the wire buffer.
 * Replaces: _pack_gradient + _pack_to_flat_buffer
 *           (axs/unified/distributed.py:70-115,147-198). */
int axs6_nf5_pack_wire(const void* x, int32_t dtype, int64_t rows, int64_t cols, int32_t block_size,
                       uint8_t* buffer, void* stream);

/* Decode a wire buffer to y [rows, cols] f32: +-codebook[code] * 2^(e-127).
 * Replaces: _unpack_from_flat_buffer + _unpack_gradient
 *           (axs/unified/distributed.py:201-232,118-144). */
int axs6_nf5_unpack_wire(const uint8_t* buffer, int64_t rows, int64_t cols, int32_t block_size, float* y,
                         void* stream);

/* AXSTensor components (exponents u8 [rows, nblk], codes and signs u8
 * [rows, nblk, block_size]; signs may be NULL) -> wire buffer.
 * Replaces: _pack_to_flat_buffer (axs/unified/distributed.py:147-198). */
int axs6_nf5_wire_from_codes(const uint8_t* exponents, const uint8_t* codes, const uint8_t* signs,
                             int64_t rows, int64_t nblk, int32_t block_size, uint8_t* buffer, void* stream);

/* Wire buffer -> AXSTensor components (signs may be NULL).
 * Replaces: _unpack_from_flat_buffer (axs/unified/distributed.py:201-232). */
int axs6_nf5_wire_to_codes(const uint8_t* buffer, int64_t rows, int64_t nblk, int32_t block_size,
                           uint8_t* exponents, uint8_t* codes, uint8_t* signs, void* stream);

/* ---- AXSBlock byte form ------------------------------------------------------
 * The concatenation of AXSBlock.to_bytes() over a tensor's blocks (blocks in
 * row-major order, the last block of a row zero-padded): per block a 2-byte
 * little-endian header e << 2 | config (config written as DENSE = 0 and
 * ignored when decoding; bits 10..15 zero), then the 6-bit codes as above,
 * four per three bytes, low bits first.  A 32-value block takes 26 bytes.
 * The same kernels as the wire format with the wider header. */

/* Bytes of the block stream of a rows x cols tensor (-1 on bad arguments). */
int64_t axs6_nf5_block_bytes(int64_t rows, int64_t cols, int32_t block_size);

/* Quantize x [rows, cols] (nearest rounding) straight into AXSBlock records.
 * Replaces: quantize_unified then AXSBlock(...).to_bytes() per block
 *           (axs/unified/quantize_unified.py:211-282, axs/core.py:97-119). */
int axs6_nf5_pack_blocks(const void* x, int32_t dtype, int64_t rows, int64_t cols, int32_t block_size,
                         uint8_t* buffer, void* stream);

/* AXSBlock records -> y [rows, cols] f32: +-codebook[code] * 2^(e-127).
 * Replaces: AXSBlock.from_bytes per block then dequantize_unified
 *           (axs/core.py:121-152, axs/unified/quantize_unified.py:285-308). */
int axs6_nf5_unpack_blocks(const uint8_t* buffer, int64_t rows, int64_t cols, int32_t block_size, float* y,
                           void* stream);

/* AXSTensor components -> AXSBlock records (signs may be NULL).
 * Replaces: AXSBlock(...).to_bytes() per block (axs/core.py:97-119). */
int axs6_nf5_blocks_from_codes(const uint8_t* exponents, const uint8_t* codes, const uint8_t* signs,
                               int64_t rows, int64_t nblk, int32_t block_size, uint8_t* buffer, void* stream);

/* AXSBlock records -> AXSTensor components (signs may be NULL).
 * Replaces: AXSBlock.from_bytes per block (axs/core.py:121-152). */
int axs6_nf5_blocks_to_codes(const uint8_t* buffer, int64_t rows, int64_t nblk, int32_t block_size,
                             uint8_t* exponents, uint8_t* codes, uint8_t* signs, void* stream);

/* ---- quantized linear ------------------------------------------------------
 * The linear contracts NF5 fake-quantized operands on fp16 MFMA.  Operands are
 * packed as fp16 rows scaled by an exact power of two (2^-shift per row, so
 * the row's largest value is <= 2^15); the GEMM epilogue restores the shifts.
 * "Kp" is K rounded up to the GEMM's contraction unit (axs6_linear_padded_k);
 * packed rows are zero beyond K.
 */

/* Contraction padding of the GEMM: K rounded up to a multiple of 64. */
int64_t axs6_linear_padded_k(int64_t k);

/* Packs rows of x [rows, cols] (cols % block_size == 0, 16-byte aligned):
 * mode 0 = values as given, 1 = NF5 FQ nearest, 2 = NF5 FQ stochastic;
 * out_f16[r, c] = fp16(v * 2^(col_exp[c] - row_shift[r])) for c < cols, zero up
 * to cols_pad (out_f16 may be NULL to compute row_shift only; col_exp may be
 * NULL).  Rows longer than 16384 f32 / 32768 16-bit values are packed in two
 * passes and need cols_pad >= 64 * ceil(cols / 64) (else
 * AXS6_ERR_UNSUPPORTED).  The FQ(x) + fp16-operand half of the fused Triton linear's tile
 * prologue (axs/unified/triton_kernels.py:152-180), run once per operand. */
int axs6_nf5_pack_rows(const void* x, int32_t dtype, int64_t rows, int64_t cols, int32_t block_size,
                       int32_t mode, uint64_t seed, uint64_t offset, const int32_t* col_exp,
                       void* out_f16, int64_t ld_out, int64_t cols_pad, int32_t* row_shift,
                       const uint64_t* seed_dev, void* stream);

/* Packing statistics of x [rows, cols] (cols % block_size == 0, 16-byte
 * aligned) without packing it: row_shift[r] = S[r] of axs6_nf5_pack_rows
 * (the largest exponent e1 of a finite nonzero block of row r plus the
 * largest col_exp over the block's columns, minus 15; 0 for a row without
 * such a block; col_exp may be NULL) and *gmax = max over rows of (largest
 * e1 + row_exp[r]) (INT_MIN when no block qualifies; row_exp may be NULL).
 * Streams the tensor in tiles instead of one workgroup per row.  The first
 * pass of the backward's dY packing (the row maxima the reference's
 * fused_fake_quantize takes per block, axs/unified/quantize_unified.py:
 * 167-175), exported so its results can be checked against
 * axs6_nf5_pack_rows; workspace: axs6_nf5_row_stats_workspace bytes. */
int64_t axs6_nf5_row_stats_workspace(int64_t rows, int64_t cols);
int axs6_nf5_row_stats(const void* x, int32_t dtype, int64_t rows, int64_t cols, int32_t block_size,
                       const int32_t* col_exp, int32_t* row_shift, const int32_t* row_exp, int32_t* gmax,
                       void* workspace, size_t workspace_bytes, void* stream);

/* out[M, N] = ldexp(A[M, Kp] . B[N, Kp]^T, row_exp[m] + col_exp[n]) + bias[n]
 * with fp16 A, B (16-byte aligned, lda/ldb multiples of 8, Kp % 64 == 0),
 * fp32 accumulation, out in out_dtype (row_exp, col_exp, bias may be NULL).
 * The contraction of the fused Triton linear (triton_kernels.py:185-282) and
 * of the backward matmuls (axs/unified/backend.py:621-671). */
int axs6_gemm_f16_nt(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M, int64_t N,
                     int64_t Kp, const int32_t* row_exp, const int32_t* col_exp, const float* bias,
                     void* out, int64_t ldo, int32_t out_dtype, void* stream);

/* Y[M, N] = FQ(X)[M, K] . FQ(W)[N, K]^T + bias, with X, W, Y of `dtype` and an
 * f32 bias (may be NULL).  K and N must be multiples of 4 (f32) or 8 (bf16,
 * f16): whole 16-byte vectors per row (a ragged last NF5 block is zero-padded
 * by the kernels, as the reference pads it).  The
 * caller provides xq_f16 [M, Kp], x_shift [M], wq_f16 [N, Kp], w_shift [N];
 * they hold the packed operands afterwards and feed the backward.
 * quantize_input = 0 packs X without fake-quantizing it.
 * Replaces: _AXSLinearUnifiedFunction.forward (axs/unified/functional_unified.py:107-131),
 *           accelerated_linear (axs/unified/backend.py:540), triton_fused_linear
 *           (axs/unified/triton_kernels.py:385). */
int axs6_nf5_linear_forward(const void* x, const void* w, const float* bias, void* y, int32_t dtype,
                            int64_t M, int64_t N, int64_t K, int32_t block_size, int32_t quantize_input,
                            void* xq_f16, int32_t* x_shift, void* wq_f16, int32_t* w_shift, void* stream);

/* Y[M, N] = FQ(X)[M, K] . FQ(W)[N, K]^T + bias in one launch, for small
 * outputs: each 32-wide K tile of X and W is NF5 fake-quantized as it is
 * loaded (the block scale and LUT step of axs6_nf5_fake_quantize, nearest
 * rounding) and contracted in fp32 (fp32 MFMA: the products of the fp32 FQ
 * values, no fp16 packing), so no quantized operand is written to memory.
 * block_size must be 32, K a multiple of 32 (zero-pad a ragged K first), x
 * and w 16-byte aligned and row-major; bias f32 (may be NULL); Y in `dtype`.
 * With quantize_input = 0, X enters the contraction as given.  For 16-bit
 * inputs the FQ values stay fp32 and only Y is rounded to `dtype`.  Meant for
 * M * N <= 131072 outputs (the Python layer dispatches there); larger
 * problems run correctly but repeat the FQ of each operand tile for every
 * output tile that reads it.
 * Replaces: triton_fused_linear / _nf5_fq_linear_kernel
 *           (axs/unified/triton_kernels.py:185-282,385-482), selected by
 *           accelerated_linear for M * N <= _FUSED_SIZE_THRESHOLD
 *           (axs/unified/backend.py:567-590, triton_kernels.py:382). */
int axs6_nf5_fused_linear(const void* x, const void* w, const float* bias, void* y, int32_t dtype,
                          int64_t M, int64_t N, int64_t K, int32_t block_size, int32_t quantize_input,
                          void* stream);

/* 1 when the caller of axs6_nf5_fused_linear does better to call
 * axs6_nf5_fused_linear_split instead -- the same results, bit for bit: x
 * whose rows neither of the single launch's LDS stagings of FQ(x) holds and
 * K >= 1024, where every workgroup would read and quantize all of x again;
 * else 0.  A host-only query (no device work), the dispatch of
 * triton_fused_linear (axs/unified/triton_kernels.py:385-482) split in two
 * launches; the reference has no counterpart. */
int32_t axs6_nf5_fused_linear_split_x(int64_t M, int64_t N, int64_t K, int32_t dtype);

/* Bytes of the x_arranged workspace axs6_nf5_fused_linear_split takes:
 * 16 * ceil(M / 16) * K floats (0 for an empty or oversized shape).  The
 * reference has no counterpart. */
int64_t axs6_nf5_fused_linear_split_workspace(int64_t M, int64_t K);

/* axs6_nf5_fused_linear in two launches: FQ(x) (x itself with
 * quantize_input = 0) is written once to x_arranged in f32, in the order the
 * contraction's 16x16x4 MFMA instructions read it, and the contraction then
 * reads it from there instead of quantizing x in every workgroup.  Same
 * arguments plus x_arranged: a 16-byte aligned device buffer of
 * axs6_nf5_fused_linear_split_workspace(M, K) bytes, overwritten.  The
 * results equal axs6_nf5_fused_linear's bit for bit wherever that takes its
 * MFMA form (every shape but the one- and two-row ones it streams, where
 * the two agree to fp32 rounding).  Replaces the same reference call as axs6_nf5_fused_linear
 * (axs/unified/triton_kernels.py:185-282,385-482). */
int axs6_nf5_fused_linear_split(const void* x, const void* w, const float* bias, void* y, float* x_arranged,
                                int32_t dtype, int64_t M, int64_t N, int64_t K, int32_t block_size,
                                int32_t quantize_input, void* stream);

/* Device workspace (bytes) axs6_nf5_linear_backward needs for the requested
 * gradients. */
size_t axs6_nf5_linear_backward_workspace(int64_t M, int64_t N, int64_t K, int32_t need_dx,
                                          int32_t need_dw, int32_t need_db);

/* Gradients of the quantized linear from dY [M, N] (`dtype`) and the packed
 * operands of the forward: dYq = NF5 FQ of dY (stochastic, blocks along N)
 * when quantize_grad, else dY; dx [M, K] (`dtype`) = dYq . FQ(W);
 * dw [N, K] f32 = dYq^T . FQ(X); db [N] f32 = column sums of dYq.  Any of dx,
 * dw, db may be NULL.  workspace: 256-byte aligned, at least
 * axs6_nf5_linear_backward_workspace(...) bytes.
 * Replaces: _AXSLinearUnifiedFunction.backward (axs/unified/functional_unified.py:134-170)
 *           with accelerated_matmul (axs/unified/backend.py:621). */
int axs6_nf5_linear_backward(const void* dy, int32_t dtype, int64_t M, int64_t N, int64_t K,
                             int32_t block_size, int32_t quantize_grad, uint64_t seed, uint64_t offset,
                             const void* xq_f16, const int32_t* x_shift, const void* wq_f16,
                             const int32_t* w_shift, void* dx, float* dw, float* db, void* workspace,
                             size_t workspace_bytes, const uint64_t* seed_dev, void* stream);

/* Largest backward workspace axs6_nf5_linear_backward_noalloc serves: the size
 * of the library's fixed per-device scratch array (64 MiB), which each device
 * the library runs on holds until the process ends. */
#define AXS6_NOALLOC_SCRATCH_BYTES (64ull << 20)

/* axs6_nf5_linear_backward without a workspace argument and without any
 * allocation: the workspace lives in the library's fixed per-device scratch
 * array (its address resolved by axs6_init or on the first call on a device).
 * Same arguments, kernels and results as axs6_nf5_linear_backward; shapes whose
 * workspace (axs6_nf5_linear_backward_workspace) exceeds
 * AXS6_NOALLOC_SCRATCH_BYTES return AXS6_ERR_UNSUPPORTED.  Every call on a
 * device shares that device's array: calls that overlap on one device (two
 * streams, two host threads) race and must be serialised by the caller.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). */
int axs6_nf5_linear_backward_noalloc(const void* dy, int32_t dtype, int64_t M, int64_t N, int64_t K,
                                     int32_t block_size, int32_t quantize_grad, uint64_t seed, uint64_t offset,
                                     const void* xq_f16, const int32_t* x_shift, const void* wq_f16,
                                     const int32_t* w_shift, void* dx, float* dw, float* db,
                                     const uint64_t* seed_dev, void* stream);

/* ---- training-step glue ----------------------------------------------------
 * Gradient unscale + overflow check + global-norm clip over a list of
 * gradient tensors: replaces the per-parameter `grad.div_(loss_scale)`, the
 * two host-synchronising isinf/isnan reductions per parameter and
 * `clip_grad_norm_(params, max_norm)` of AXSTrainingPipelineUnified.training_step
 * (axs/unified/training_unified.py:224-257, _check_overflow :287-292):
 *   every element g *= fl(1 / loss_scale) (the fp32 reciprocal, rounded to the
 *   tensor dtype: what torch's grad.div_(loss_scale) computes on the GPU);
 *   result[0] = sqrt(sum of g^2 over all tensors), summed in a fixed order;
 *   result[1] = min(max_norm / (result[0] + 1e-6), 1)  (NaN stays NaN);
 *   result[2] = number of non-finite values after the division;
 *   with clip != 0, when result[2] == 0 and result[1] < 1: g *= result[1].
 * grads, numel and dtypes are HOST arrays of `count` entries (device pointers,
 * element counts, dtype codes; tensors contiguous and element-aligned).
 * partials: device floats, at least axs6_multi_tensor_workspace(numel, count)
 * of them; result: 3 device floats.  Asynchronous: no host synchronisation,
 * no allocation; the caller reads `result` when it needs the values. */
int64_t axs6_multi_tensor_workspace(const int64_t* numel, int32_t count);
int axs6_multi_tensor_unscale_clip(void* const* grads, const int64_t* numel, const int32_t* dtypes, int32_t count,
                                   float loss_scale, float max_norm, int32_t clip, float* partials,
                                   int64_t partials_len, float* result, void* stream);

/* ---- LayerNorm -------------------------------------------------------------
 * F.layer_norm of AXSLayerNormUnified.forward (axs/unified/modules_unified.py:
 * 141-144) and its autograd backward, over rows of `cols` contiguous values
 * (the normalized dims flattened); x, y, dy, dx, gamma, beta of `dtype`,
 * statistics and parameter gradients in float32:
 *   mean = sum x / cols, var = sum (x - mean)^2 / cols, rstd = 1 / sqrt(var + eps),
 *   y = (x - mean) * rstd * gamma + beta                 (gamma, beta NULL: 1, 0);
 *   dx = rstd * (g - (sum g + xhat * sum g * xhat) / cols), g = dy * gamma,
 *   dgamma = sum over rows of dy * xhat, dbeta = sum over rows of dy.
 * mean and rstd (rows floats each) are written by the forward when not NULL
 * and read by the backward; dgamma / dbeta may be NULL.  The backward needs
 * axs6_layer_norm_backward_workspace(rows, cols) bytes of device workspace.
 * Deterministic (fixed reduction orders), asynchronous, no allocation. */
int axs6_layer_norm_forward(const void* x, int32_t dtype, int64_t rows, int64_t cols, const void* gamma,
                            const void* beta, float eps, void* y, float* mean, float* rstd, void* stream);
int64_t axs6_layer_norm_backward_workspace(int64_t rows, int64_t cols);
int axs6_layer_norm_backward(const void* dy, const void* x, int32_t dtype, int64_t rows, int64_t cols,
                             const float* mean, const float* rstd, const void* gamma, void* dx, float* dgamma,
                             float* dbeta, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AXS6_H */
