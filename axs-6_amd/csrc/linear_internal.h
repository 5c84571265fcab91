// Launchers shared by the quantized-linear translation units.
#pragma once

#include "axs6_internal.h"

namespace axs6 {

// Row pack: per row r of x [rows, cols] (cols % block == 0, 16-byte aligned
// rows), v = FQ(x) (or x when !fake_quant), and
//   out[r, c] = fp16(v * 2^(colx[c] - S[r]))      for c < cols
//   out[r, c] = 0                                  for cols <= c < cols_pad
// with S[r] = max_c(e1(block of c) + colx[c]) - 15, where 2^e1 bounds the
// block's magnitudes, so |out| <= 2^15 < fp16 max.  S[r] goes to s_out.
// rmax_out[r] (optional) = max block e1 of the row (colx ignored);
// gmax (optional) receives atomicMax(rmax + rowx[r]).
// `out` may be null (statistics only).
struct PackRowsArgs {
    const void* x; int dtype; int64_t rows; int64_t cols; int block;
    bool fake_quant; bool stochastic; uint64_t seed; uint64_t offset;
    const uint64_t* seed_dev;       // nullable: added to seed when the kernel runs
    const int32_t* colx;            // nullable
    _Float16* out; int64_t ld_out; int64_t cols_pad;
    int32_t* s_out;                 // [rows]
    int32_t* rmax_out;              // nullable
    const int32_t* rowx; int32_t* gmax;  // nullable pair
};
int launch_pack_rows(const PackRowsArgs& a, const DeviceTables& t, hipStream_t st);
// Two independent row packs in one launch when they share dtype, mode and
// row length class (the forward's X and W); otherwise two launches.
int launch_pack_rows2(const PackRowsArgs& a, const PackRowsArgs& b, const DeviceTables& t, hipStream_t st);

// Transposed global pack: out[c, r] = fp16(FQ(x)[r, c] * 2^(rowx[r] - (*gmax - 15)))
// for c < cols, r < rows; zero for rows <= r < pad_to(rows, 64) (ld_out >= that).
// FQ uses the same dither counters as pack_rows on the same x, seed and offset.
// Optional column partial sums of FQ(x): partial[chunk, c] over the 64 rows of
// chunk, in a fixed order.  gmax may be null (shift 0).
// Also, with out_r: the row-major operand out_r[r, c] = fp16(FQ(x)[r, c] *
// 2^(colx_r[c] - shift_r[r])) for r < rows, zero for cols <= c < pad_to(cols, 64)
// -- what pack_rows writes, with the row shifts taken from a statistics-only
// pack_rows pass (mode raw, no output).
struct PackTArgs {
    const void* x; int dtype; int64_t rows; int64_t cols; int block;
    bool fake_quant; bool stochastic; uint64_t seed; uint64_t offset;
    const uint64_t* seed_dev;       // nullable
    const int32_t* rowx;            // nullable (0)
    const int32_t* gmax;            // device scalar, nullable
    _Float16* out; int64_t ld_out;  // out nullable
    _Float16* out_r; int64_t ld_r;  // out_r nullable
    const int32_t* colx_r;          // nullable (0)
    const int32_t* shift_r;         // required with out_r
    float* partial;                 // nullable
    // nullable: per-band maxima of the statistics pass (row_stats_final_bands),
    // folded into the tensor-wide maximum in place of *gmax and written to gmax_out
    const int32_t* gtile = nullptr; int64_t ngtile = 0; int32_t* gmax_out = nullptr;
};
int launch_pack_t(const PackTArgs& a, const DeviceTables& t, hipStream_t st);

// Row statistics of x (block exponents only): shift[r] = max over the row's
// finite nonzero blocks of (e1 + max colx over the block) - 15 (0 if none),
// and gmax = max over rows of (max block e1 + rowx[r]) (INT_MIN if none) --
// the shifts pack_rows derives.  scratch: 2 * rows int32 of device memory.
struct RowStatsArgs {
    const void* x; int dtype; int64_t rows; int64_t cols; int block;
    const int32_t* colx;            // nullable (0)
    int32_t* shift;                 // nullable
    const int32_t* rowx;            // nullable (0)
    int32_t* gmax;                  // nullable
    int32_t* scratch;               // [2 * row_stats_col_tiles(cols) * rows]
    // with gtile and row_stats_final_bands(...) > 0: shift is written by the one
    // pass, gmax is not, and gtile[band] receives each band's maximum (see PackTArgs)
    int32_t* gtile = nullptr;
};
// Row bands of the one-pass statistics (rows of at most 256 values), 0 when
// the rows are longer (two passes: tiles, then a folding launch).
int64_t row_stats_final_bands(int64_t rows, int64_t cols, int dtype);
// column tiles of the statistics pass: its scratch holds two ints per tile and row
int64_t row_stats_col_tiles(int64_t cols);
struct TransposeF16;
// With ta (and tb), the transposes of launch_transpose_f16 (without db) run
// in the statistics launch when they take 128 x 128 tiles, else after it.
int launch_row_stats(const RowStatsArgs& a, const DeviceTables& t, hipStream_t st,
                     const TransposeF16* ta = nullptr, const TransposeF16* tb = nullptr);

int64_t pack_global_chunks(int64_t rows);

// db[c] = sum_k partial[k, c], k in order.
int launch_reduce_partials(const float* partial, int64_t chunks, int64_t cols, float* out, hipStream_t st);

// out[c, r] = in[r, c] for r < rows, c < out_rows; zero for rows <= r < rows_pad.
struct TransposeF16 {
    const _Float16* in; int64_t rows; int64_t cols; int64_t ld_in;
    _Float16* out; int64_t out_rows; int64_t rows_pad; int64_t ld_out;
};
// a, and b when not null, in one launch; with db (and partial), the same
// launch also writes db[c] = sum_k partial[k, c] (launch_reduce_partials)
int launch_transpose_f16(const TransposeF16& a, const TransposeF16* b, hipStream_t st,
                         const float* partial = nullptr, int64_t chunks = 0, int64_t cols = 0, float* db = nullptr);

// *p = INT32_MIN (graph-capture safe: a kernel, not a memset).
int launch_init_gmax(int32_t* p, hipStream_t st);

// C[M, N] = epilogue(A[M, Kp] . B[N, Kp]^T); fp16 operands, fp32 accumulate.
// Epilogue: v = ldexp(acc, row_exp[m] + col_exp[n] + (glob ? *glob + glob_add : 0)) + bias[n].
// With split_partial (device memory of split_bytes >= gemm_split_bytes(M, N,
// Kp)), a GEMM with few output tiles and a long contraction splits K over
// gemm_split_count(M, N, Kp) workgroups per tile, writing fp32 partial tiles
// that a second kernel sums in a fixed order before the epilogue.
struct GemmArgs {
    const _Float16* A; int64_t lda; const _Float16* B; int64_t ldb;
    int64_t M; int64_t N; int64_t Kp;
    const int32_t* row_exp; const int32_t* col_exp;
    const int32_t* glob_exp; int32_t glob_add;
    const float* bias;
    void* out; int64_t ldo; int out_dtype;
    float* split_partial = nullptr; size_t split_bytes = 0;
    // when the GEMM splits K: red_out[c] = sum over red_chunks rows of
    // red_partial[., c] (launch_reduce_partials) in the split reduction's launch
    const float* red_partial = nullptr; int64_t red_chunks = 0; int64_t red_cols = 0; float* red_out = nullptr;
};
int launch_gemm_f16(const GemmArgs& g, hipStream_t st);
// Whether launch_gemm_f16(g) splits K (and so runs a reduction launch after the GEMM).
bool gemm_splits(const GemmArgs& g);
// a and b (independent; at most one of them splitting K, since split-K partials
// share one buffer) in one launch when they take the same small-tile kernel
// configuration (gemm_pairs), else one launch each; each split's reduction
// follows.  b's red_* job runs in b's split reduction, or in the pair launch.
int launch_gemm_pair(const GemmArgs& a, const GemmArgs& b, hipStream_t st);
bool gemm_pairs(const GemmArgs& a, const GemmArgs& b);
int gemm_split_count(int64_t M, int64_t N, int64_t Kp);
size_t gemm_split_bytes(int64_t M, int64_t N, int64_t Kp);

constexpr int64_t kGemmK = 64;   // contraction padding unit
inline int64_t pad_to(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

}  // namespace axs6
