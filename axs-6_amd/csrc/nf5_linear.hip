// Quantized linear (forward, backward) and plain matmul: host-side
// composition of the packing kernels and the fp16 MFMA GEMM, exported
// through the C ABI of include/axs6.h.
//
// Forward  Y = FQ(X) FQ(W)^T + b:
//   pack_rows(X), pack_rows(W) in one launch -> Xq16 [M, Kp], sx[M] and
//   Wq16 [N, Kp], sw[N]                       (FQ + row scale, one HBM pass)
//   GEMM(Xq16, Wq16) with epilogue 2^(sx[m] + sw[n]) and + b
// Xq16/sx/Wq16/sw are caller-owned and reused by the backward.
//
// Backward (dYq = stochastic FQ(dY) when quantize_grad, else dY):
//   row_stats(dY):    the row shifts t[m] of the dX operand (with the weight's
//                     row exponents sw folded in per column) and the
//                     tensor-wide shift G of the dW operand (max over rows of
//                     the row maxima + sx[m]) -- block exponents only, no FQ
//                     values, streamed over 2-D tiles that store per-tile
//                     row maxima, folded per row in order by a second kernel;
//   pack_t(dY):       one pass over 64x64 tiles computes dYq once and writes
//                     A1 [M, Np] = dYq * 2^(sw[n] - t[m]) (row-major, for dX),
//                     A2T [N, Mp] = (dYq * 2^(sx[m] - G))^T (for dW, transposed
//                     through LDS) and the fixed-order column partials for db;
//   dX = dYq FQ(W):   transpose Wq16 -> [Kp, Np], GEMM(A1, WqT), epilogue 2^t[m];
//   dW = dYq^T FQ(X): transpose Xq16 -> [Kp, Mp], GEMM(A2T, XqT), epilogue 2^G;
//   db = reduce of the partials (fixed order).
#include <string.h>

#include <mutex>

#include "linear_internal.h"

namespace axs6 {
namespace {

constexpr size_t kAlign = 256;
inline size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct BwdLayout {
    bool dx, dw, db;   // which gradients the layout serves
    size_t gmax, t, stats, gtile, a1, wqt, a2t, xqt, partial, splitk, splitk_bytes, total;
    int64_t bands;   // row bands of the one-pass statistics (0: two passes)
};

BwdLayout bwd_layout(int64_t M, int64_t N, int64_t K, bool dx, bool dw, bool db, int dtype) {
    const int64_t Kp = pad_to(K, kGemmK), Np = pad_to(N, kGemmK), Mp = pad_to(M, kGemmK);
    BwdLayout L{};
    L.dx = dx;
    L.dw = dw;
    L.db = db;
    size_t off = 0;
    auto take = [&](size_t bytes) { size_t o = off; off = align_up(off + bytes); return o; };
    L.gmax = take(sizeof(int32_t));
    L.t = take(sizeof(int32_t) * (size_t)M);
    L.stats = take(2 * sizeof(int32_t) * (size_t)row_stats_col_tiles(N) * (size_t)M);
    L.bands = (dx || dw) ? row_stats_final_bands(M, N, dtype) : 0;
    L.gtile = L.bands ? take(sizeof(int32_t) * (size_t)L.bands) : 0;
    L.a1 = dx ? take(2 * (size_t)M * Np) : 0;
    L.wqt = dx ? take(2 * (size_t)Kp * Np) : 0;
    L.a2t = dw ? take(2 * (size_t)N * Mp) : 0;
    L.xqt = dw ? take(2 * (size_t)Kp * Mp) : 0;
    L.partial = db ? take(sizeof(float) * (size_t)pack_global_chunks(M) * N) : 0;
    // split-K partial tiles, shared by the dX and dW GEMMs (they run in order)
    const size_t sx = dx ? gemm_split_bytes(M, K, Np) : 0, sw = dw ? gemm_split_bytes(N, K, Mp) : 0;
    L.splitk_bytes = sx > sw ? sx : sw;
    L.splitk = L.splitk_bytes ? take(L.splitk_bytes) : 0;
    L.total = off;
    return L;
}

int check_dims(const char* fn, int64_t M, int64_t N, int64_t K, int block, int dtype) {
    if (!valid_dtype(dtype)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: unknown dtype code %d", fn, dtype);
    if (!valid_block(block)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: block_size must be 8, 16 or 32 (got %d)", fn, block);
    if (M < 0 || N < 0 || K < 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: negative dimension", fn);
    // whole 16-byte vectors per row of X, W and dY (a ragged last NF5 block is
    // zero-padded by the kernels, as the reference pads it)
    const int64_t vm = dtype == AXS6_F32 ? 4 : 8;
    if (K % vm != 0 || N % vm != 0)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: K (%lld) and N (%lld) must be multiples of %lld "
                    "(pad them with zeros first)", fn, (long long)K, (long long)N, (long long)vm);
    if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: dimension too large", fn);
    return AXS6_OK;
}

}  // namespace
}  // namespace axs6

using namespace axs6;

extern "C" int64_t axs6_linear_padded_k(int64_t k) { return pad_to(k, kGemmK); }

extern "C" int axs6_nf5_pack_rows(const void* x, int32_t dtype, int64_t rows, int64_t cols, int32_t block_size,
                                  int32_t mode, uint64_t seed, uint64_t offset, const int32_t* col_exp,
                                  void* out_f16, int64_t ld_out, int64_t cols_pad, int32_t* row_shift,
                                  const uint64_t* seed_dev, void* stream) {
    const char* fn = "axs6_nf5_pack_rows";
    if (!valid_dtype(dtype)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: unknown dtype code %d", fn, dtype);
    if (!valid_block(block_size)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: block_size must be 8, 16 or 32", fn);
    if (mode < 0 || mode > 2) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: mode must be 0 (raw), 1 (nearest) or 2 (stochastic)", fn);
    if (rows < 0 || cols < 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: negative shape", fn);
    if (rows == 0) return AXS6_OK;
    if (!x || !row_shift) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    if (out_f16 && ld_out < cols_pad)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: ld_out (%lld) is smaller than cols_pad (%lld)", fn,
                    (long long)ld_out, (long long)cols_pad);
    DeviceTables t;
    int rc = device_tables(&t);
    if (rc) return rc;
    PackRowsArgs a{x, dtype, rows, cols, block_size, mode != 0, mode == 2, seed, offset, seed_dev, col_exp,
                   (_Float16*)out_f16, ld_out, cols_pad, row_shift, nullptr, nullptr, nullptr};
    return launch_pack_rows(a, t, (hipStream_t)stream);
}

extern "C" int axs6_gemm_f16_nt(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M, int64_t N,
                                int64_t Kp, const int32_t* row_exp, const int32_t* col_exp, const float* bias,
                                void* out, int64_t ldo, int32_t out_dtype, void* stream) {
    const char* fn = "axs6_gemm_f16_nt";
    if (!valid_dtype(out_dtype)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: unknown dtype code %d", fn, out_dtype);
    if (M < 0 || N < 0 || Kp < 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: negative dimension", fn);
    if (M == 0 || N == 0) return AXS6_OK;
    if (!a || !b || !out) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    GemmArgs g{(const _Float16*)a, lda, (const _Float16*)b, ldb, M, N, Kp, row_exp, col_exp, nullptr, 0, bias,
               out, ldo, out_dtype};
    return launch_gemm_f16(g, (hipStream_t)stream);
}

extern "C" int64_t axs6_nf5_row_stats_workspace(int64_t rows, int64_t cols) {
    if (rows < 0 || cols < 0) return 0;
    return 2 * (int64_t)sizeof(int32_t) * row_stats_col_tiles(cols) * rows;
}

extern "C" int axs6_nf5_row_stats(const void* x, int32_t dtype, int64_t rows, int64_t cols, int32_t block_size,
                                  const int32_t* col_exp, int32_t* row_shift, const int32_t* row_exp, int32_t* gmax,
                                  void* workspace, size_t workspace_bytes, void* stream) {
    const char* fn = "axs6_nf5_row_stats";
    if (!valid_dtype(dtype)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: unknown dtype code %d", fn, dtype);
    if (!valid_block(block_size))
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: block_size must be 8, 16 or 32 (got %d)", fn, block_size);
    if (rows < 0 || cols < 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: negative dimension", fn);
    if (rows == 0 || cols == 0) return AXS6_OK;
    if (!x || (!row_shift && !gmax)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    const int64_t need = axs6_nf5_row_stats_workspace(rows, cols);
    if (!workspace || (int64_t)workspace_bytes < need || (uintptr_t)workspace % 16)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: workspace of %lld bytes (16-byte aligned) required", fn,
                    (long long)need);
    DeviceTables t;
    int rc = device_tables(&t);
    if (rc) return rc;
    RowStatsArgs s{x, dtype, rows, cols, block_size, col_exp, row_shift, row_exp, gmax, (int32_t*)workspace};
    return launch_row_stats(s, t, (hipStream_t)stream);
}

extern "C" int axs6_nf5_linear_forward(const void* x, const void* w, const float* bias, void* y, int32_t dtype,
                                       int64_t M, int64_t N, int64_t K, int32_t block_size,
                                       int32_t quantize_input, void* xq_f16, int32_t* x_shift, void* wq_f16,
                                       int32_t* w_shift, void* stream) {
    const char* fn = "axs6_nf5_linear_forward";
    int rc = check_dims(fn, M, N, K, block_size, dtype);
    if (rc) return rc;
    if (M == 0 || N == 0) return AXS6_OK;
    if (!x || !w || !y || !xq_f16 || !x_shift || !wq_f16 || !w_shift)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    DeviceTables t;
    if ((rc = device_tables(&t))) return rc;
    hipStream_t st = (hipStream_t)stream;
    const int64_t Kp = pad_to(K, kGemmK);
    PackRowsArgs px{x, dtype, M, K, block_size, quantize_input != 0, false, 0, 0, nullptr, nullptr,
                    (_Float16*)xq_f16, Kp, Kp, x_shift, nullptr, nullptr, nullptr};
    PackRowsArgs pw{w, dtype, N, K, block_size, true, false, 0, 0, nullptr, nullptr,
                    (_Float16*)wq_f16, Kp, Kp, w_shift, nullptr, nullptr, nullptr};
    if ((rc = launch_pack_rows2(px, pw, t, st))) return rc;
    GemmArgs g{(const _Float16*)xq_f16, Kp, (const _Float16*)wq_f16, Kp, M, N, Kp, x_shift, w_shift, nullptr, 0,
               bias, y, N, dtype};
    return launch_gemm_f16(g, st);
}

extern "C" size_t axs6_nf5_linear_backward_workspace(int64_t M, int64_t N, int64_t K, int32_t need_dx,
                                                     int32_t need_dw, int32_t need_db) {
    if (M < 0 || N < 0 || K < 0) return 0;
    return bwd_layout(M, N, K, need_dx != 0 && K > 0, need_dw != 0 && K > 0, need_db != 0, AXS6_F32).total;
}

namespace axs6 {
namespace {

struct BwdCall {
    const void* dy; int32_t dtype; int64_t M, N, K; int32_t block_size, quantize_grad; uint64_t seed, offset;
    const void* xq_f16; const int32_t* x_shift; const void* wq_f16; const int32_t* w_shift;
    void* dx; float* dw; float* db; const uint64_t* seed_dev; void* stream;
};

// Argument checks shared by both backward entry points; *run is false when
// there is nothing to compute (empty shapes, no gradient requested).
int bwd_check(const char* fn, const BwdCall& c, bool* run, BwdLayout* L) {
    *run = false;
    int rc = check_dims(fn, c.M, c.N, c.K, c.block_size, c.dtype);
    if (rc) return rc;
    // with K == 0, dX [M, 0] and dW [N, 0] are empty; db is still the column sums of dYq
    const bool need_dx = c.dx != nullptr && c.K > 0, need_dw = c.dw != nullptr && c.K > 0, need_db = c.db != nullptr;
    if (c.M == 0 || c.N == 0 || (!need_dx && !need_dw && !need_db)) return AXS6_OK;
    if (!c.dy) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null dy", fn);
    if ((need_dx && (!c.wq_f16 || !c.w_shift)) || (need_dw && (!c.xq_f16 || !c.x_shift)))
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: packed operands from the forward are required", fn);
    *L = bwd_layout(c.M, c.N, c.K, need_dx, need_dw, need_db, c.dtype);
    *run = true;
    return AXS6_OK;
}

// The backward's launches with `workspace` laid out by L (every byte a kernel
// reads is written earlier in the same call, so nothing needs clearing).
int bwd_run(const BwdCall& c, const BwdLayout& L, char* ws) {
    const void* dy = c.dy;
    const int32_t dtype = c.dtype, block_size = c.block_size;
    const int64_t M = c.M, N = c.N, K = c.K;
    const int32_t* x_shift = c.x_shift;
    const int32_t* w_shift = c.w_shift;
    float* db = c.db;
    const bool need_dx = L.dx, need_dw = L.dw, need_db = L.db;
    int rc;
    DeviceTables t;
    if ((rc = device_tables(&t))) return rc;
    hipStream_t st = (hipStream_t)c.stream;
    const int64_t Kp = pad_to(K, kGemmK), Np = pad_to(N, kGemmK), Mp = pad_to(M, kGemmK);
    int32_t* gmax = (int32_t*)(ws + L.gmax);
    int32_t* tshift = (int32_t*)(ws + L.t);
    const bool fq = c.quantize_grad != 0;

    _Float16* wqt = need_dx ? (_Float16*)(ws + L.wqt) : nullptr;
    _Float16* xqt = need_dw ? (_Float16*)(ws + L.xqt) : nullptr;
    float* partial = need_db ? (float*)(ws + L.partial) : nullptr;
    float* splitk = L.splitk_bytes ? (float*)(ws + L.splitk) : nullptr;
    GemmArgs gx{(const _Float16*)(ws + L.a1), Np, wqt, Np, M, K, Np, tshift, nullptr, nullptr, 0, nullptr,
                c.dx, K, dtype, splitk, L.splitk_bytes};
    GemmArgs gw{(const _Float16*)(ws + L.a2t), Mp, xqt, Mp, N, K, Mp, nullptr, nullptr, gmax, -15, nullptr, c.dw, K,
                AXS6_F32, splitk, L.splitk_bytes};
    // contraction-contiguous copies of the forward's operands (WqT for dX,
    // XqT for dW): they depend only on the forward, so they ride in the
    // statistics launch -- unless db needs the launch after the packing pass
    // (below) and the dW GEMM has no split-K reduction launch to carry it
    const TransposeF16 tw{(const _Float16*)c.wq_f16, N, Kp, Kp, wqt, Kp, Np, Np};
    const TransposeF16 tx{(const _Float16*)c.xq_f16, M, Kp, Kp, xqt, Kp, Mp, Mp};
    const TransposeF16* t0 = need_dx ? &tw : &tx;
    const TransposeF16* t1 = need_dx && need_dw ? &tx : nullptr;
    // db rides in the dW GEMM's split reduction, or in the dX + dW pair launch
    const bool db_in_dw = need_db && need_dw && (gemm_splits(gw) || (need_dx && gemm_pairs(gx, gw)));
    const bool t_early = (need_dx || need_dw) && (!need_db || db_in_dw);

    // rows of at most 256 values: one statistics launch writes the row shifts
    // and per-band maxima, which the packing pass folds into G
    int32_t* gtile = L.bands ? (int32_t*)(ws + L.gtile) : nullptr;
    if (need_dx || need_dw) {
        RowStatsArgs s{dy, dtype, M, N, block_size, need_dx ? w_shift : nullptr, tshift,
                       need_dw ? x_shift : nullptr, need_dw ? gmax : nullptr, (int32_t*)(ws + L.stats), gtile};
        if ((rc = launch_row_stats(s, t, st, t_early ? t0 : nullptr, t_early ? t1 : nullptr))) return rc;
    }
    if (need_dx || need_dw || need_db) {
        const bool fold = gtile && need_dw;
        PackTArgs p{dy, dtype, M, N, block_size, fq, fq, c.seed, c.offset, c.seed_dev, x_shift,
                    need_dw && !fold ? gmax : nullptr,
                    need_dw ? (_Float16*)(ws + L.a2t) : nullptr, Mp,
                    need_dx ? (_Float16*)(ws + L.a1) : nullptr, Np, w_shift, tshift, partial,
                    fold ? gtile : nullptr, fold ? L.bands : 0, fold ? gmax : nullptr};
        if ((rc = launch_pack_t(p, t, st))) return rc;
    }
    // the bias gradient's ordered reduction of the pack's partial sums: in the
    // dW GEMM's split-K reduction launch or the dX + dW pair launch, else in
    // the transposes' launch (or alone when no operand is transposed)
    if (!t_early && (need_dx || need_dw)) {
        if ((rc = launch_transpose_f16(*t0, t1, st, partial, pack_global_chunks(M), N, db))) return rc;
    } else if (need_db && !db_in_dw && !(need_dx || need_dw) &&
               (rc = launch_reduce_partials(partial, pack_global_chunks(M), N, db, st))) {
        return rc;
    }
    if (db_in_dw) {
        gw.red_partial = partial;
        gw.red_chunks = pack_global_chunks(M);
        gw.red_cols = N;
        gw.red_out = db;
    }
    // dX and dW are independent: one launch when they share a configuration
    if (need_dx && need_dw) {
        if ((rc = launch_gemm_pair(gx, gw, st))) return rc;
    } else if (need_dx) {
        if ((rc = launch_gemm_f16(gx, st))) return rc;
    } else if (need_dw) {
        if ((rc = launch_gemm_f16(gw, st))) return rc;
    }
    return AXS6_OK;
}

// Scratch of the allocation-free backward: one instance per device, resolved
// to its device address once per device (hipGetSymbolAddress with that device
// current).  In host code the array's name is only a host-side handle; kernels
// receive the resolved address.  Every call on a device shares the array, so
// calls that overlap on one device race.
static __device__ __align__(256) unsigned char scratch[AXS6_NOALLOC_SCRATCH_BYTES];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch[kScratchDevices];

int noalloc_scratch(char** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0) return fail(AXS6_ERR_NO_DEVICE, "no current HIP device: %s", hipGetErrorString(e));
    if (dev >= kScratchDevices) return fail(AXS6_ERR_UNSUPPORTED, "device ordinal %d beyond %d", dev, kScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        char* ptr = nullptr;
        if ((e = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch))) != hipSuccess || !ptr)
            return fail(AXS6_ERR_HIP, "scratch address lookup on device %d failed: %s", dev, hipGetErrorString(e));
        g_scratch[dev] = ptr;
    }
    *out = g_scratch[dev];
    return AXS6_OK;
}

}  // namespace

// Resolves the current device's scratch address (the library's init call).
int init_noalloc_scratch() {
    char* p;
    return noalloc_scratch(&p);
}

}  // namespace axs6

extern "C" int axs6_nf5_linear_backward(const void* dy, int32_t dtype, int64_t M, int64_t N, int64_t K,
                                        int32_t block_size, int32_t quantize_grad, uint64_t seed, uint64_t offset,
                                        const void* xq_f16, const int32_t* x_shift, const void* wq_f16,
                                        const int32_t* w_shift, void* dx, float* dw, float* db, void* workspace,
                                        size_t workspace_bytes, const uint64_t* seed_dev, void* stream) {
    const char* fn = "axs6_nf5_linear_backward";
    const BwdCall c{dy, dtype, M, N, K, block_size, quantize_grad, seed, offset, xq_f16, x_shift, wq_f16, w_shift,
                    dx, dw, db, seed_dev, stream};
    bool run;
    BwdLayout L;
    int rc = bwd_check(fn, c, &run, &L);
    if (rc || !run) return rc;
    if (!workspace || workspace_bytes < L.total || (uintptr_t)workspace % kAlign)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: workspace of %zu bytes (256-byte aligned) required, got %zu",
                    fn, L.total, workspace_bytes);
    return bwd_run(c, L, (char*)workspace);
}

extern "C" int axs6_nf5_linear_backward_noalloc(const void* dy, int32_t dtype, int64_t M, int64_t N, int64_t K,
                                                int32_t block_size, int32_t quantize_grad, uint64_t seed,
                                                uint64_t offset, const void* xq_f16, const int32_t* x_shift,
                                                const void* wq_f16, const int32_t* w_shift, void* dx, float* dw,
                                                float* db, const uint64_t* seed_dev, void* stream) {
    const char* fn = "axs6_nf5_linear_backward_noalloc";
    const BwdCall c{dy, dtype, M, N, K, block_size, quantize_grad, seed, offset, xq_f16, x_shift, wq_f16, w_shift,
                    dx, dw, db, seed_dev, stream};
    bool run;
    BwdLayout L;
    int rc = bwd_check(fn, c, &run, &L);
    if (rc || !run) return rc;
    if (L.total > (size_t)AXS6_NOALLOC_SCRATCH_BYTES)
        return fail(AXS6_ERR_UNSUPPORTED,
                    "%s: this shape needs %zu bytes of scratch, beyond the library's fixed %llu bytes; "
                    "use axs6_nf5_linear_backward with a caller workspace", fn, L.total,
                    (unsigned long long)AXS6_NOALLOC_SCRATCH_BYTES);
    char* ws;
    if ((rc = noalloc_scratch(&ws))) return rc;
    return bwd_run(c, L, ws);
}
