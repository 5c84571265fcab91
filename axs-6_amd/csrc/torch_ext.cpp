// Torch extension `axs._C`: the host side of the NF5 fake-quantize and the
// AXS-6 quantized linear in C++ over the C ABI of libaxs6.so
// (include/axs6.h).
//
// The fake-quantize with its straight-through gradient (the reference's
// _FusedQuantizeSTE, functional_unified.py:38-60) is a C++ autograd node too,
// so a call costs one node and one library call, with no Python in between.
//
// The reference's _AXSLinearUnifiedFunction (axs/unified/functional_unified.py:
// 107-170) is a Python autograd Function.  Here the same operation is a C++
// autograd node: shape handling, output and workspace allocation, the dither
// seed and the two library calls run without Python, and the autograd engine
// calls the backward directly.  The same forward/backward helpers are exported
// for the Python-level wrappers (axs.unified.hip_linear), so every path shares
// one implementation.
//
// Semantics (as the Python wrappers documented them before this extension):
//   * input (*, K) and weight (N, K) on one GPU; float32, bfloat16 or float16
//     are computed in their own type, any other floating dtype in float32
//     and returned (Y, dX) in its own type;
//   * a bias broadcasts as in F.linear (N values, or one); other lengths raise;
//   * a K or N that is not a multiple of 4 (float32) or 8 (bfloat16, float16)
//     is zero-padded on the device to one (NF5 pads the last block with
//     zeros, so nothing changes); other ragged lengths go to the kernels as
//     they are, which zero-pad the last block themselves;
//   * views whose data pointer is not 16-byte aligned are copied (the packing
//     kernels load 16-byte vectors);
//   * K == 0 gives the bias (or zeros) like F.linear, M == 0 empty outputs and
//     zero dW / db;
//   * dW is float32 and then cast to the weight's dtype; db is float32;
//   * the stochastic rounding of dY draws its seed from torch's default CPU
//     generator (torch.randint(0, 2**62, (1,))), and while the current stream
//     records a graph it adds a per-device counter read on the device, which
//     the graph advances once (after its first such call), so replays draw
//     fresh dither values.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPGraphsC10Utils.h>
#include <c10/hip/HIPStream.h>

#include <cstdint>
#include <mutex>
#include <optional>
#include <unordered_map>

#include "axs6.h"

namespace {

using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

int dtype_code(at::ScalarType t) {
    switch (t) {
        case at::kFloat: return AXS6_F32;
        case at::kBFloat16: return AXS6_BF16;
        case at::kHalf: return AXS6_F16;
        default: return -1;
    }
}

at::ScalarType compute_dtype(at::ScalarType t) { return dtype_code(t) >= 0 ? t : at::kFloat; }

void check_rc(int rc, const char* fn) {
    TORCH_CHECK(rc == 0, fn, " failed (status ", rc, "): ", axs6_last_error());
}

void require_device(const at::Tensor& t, const char* fn) {
    TORCH_CHECK(t.is_cuda(), fn, " requires a CUDA (ROCm/HIP) device tensor, got device ", t.device());
}

void* stream_of(const at::Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

int64_t pad_amount(int64_t n, int64_t mult) { return (mult - n % mult) % mult; }

// t viewed as (rows, cols) over its last dim (also when cols is 0).
at::Tensor rows2d(const at::Tensor& t, int64_t cols) {
    int64_t rows = 1;
    for (int64_t d = 0; d + 1 < t.dim(); ++d) rows *= t.size(d);
    return t.reshape({rows, cols});
}

// Row lengths the kernels take without a copy: whole 16-byte vectors (4
// float32 or 8 bfloat16 / float16 values); a ragged last NF5 block is
// zero-padded by the kernels themselves.
int64_t vec_multiple(at::ScalarType dtype) { return dtype == at::kFloat ? 4 : 8; }

at::Tensor pad_last(const at::Tensor& t, int64_t mult) {
    const int64_t p = pad_amount(t.size(-1), mult);
    return p ? at::constant_pad_nd(t, {0, p}) : t;
}

at::Tensor pad_rows(const at::Tensor& t, int64_t mult) {
    const int64_t p = pad_amount(t.size(0), mult);
    return p ? at::constant_pad_nd(t, {0, 0, 0, p}) : t;
}

at::Tensor dense(const at::Tensor& t) {
    at::Tensor c = t.contiguous();
    return reinterpret_cast<uintptr_t>(c.data_ptr()) % 16 == 0 ? c : c.clone(at::MemoryFormat::Contiguous);
}

// The bias as F.linear broadcasts it over the N output features: one value,
// or N values as (N,) or (1, N); anything else raises, as F.linear does (a
// shorter bias would otherwise be read past its end by the kernels).
at::Tensor bias_vector(const at::Tensor& bias, int64_t N, const char* fn) {
    const int64_t n = bias.numel();
    if (n == 1 && N != 1) return bias.reshape({1}).expand({N});
    TORCH_CHECK(n == N && (bias.dim() == 1 || (bias.dim() == 2 && bias.size(0) == 1)), fn, ": bias of shape ",
                bias.sizes(), " does not broadcast to the ", N, " output features");
    return bias.reshape({N});
}

// Floating dtypes other than the three computed natively (float64) come back
// in their own type, as the reference's F.linear on their fake-quantized
// values returns them; the kernels compute them in float32.
at::Tensor to_input_dtype(const at::Tensor& y, at::ScalarType in) {
    return (y.scalar_type() != in && at::isFloatingType(in)) ? y.to(in) : y;
}

std::vector<int64_t> lead_shape(at::IntArrayRef shape, int64_t last) {
    std::vector<int64_t> s(shape.begin(), shape.end());
    if (s.empty()) s.push_back(last);
    else s.back() = last;
    return s;
}

// ---- dither seeds -----------------------------------------------------------

// Per-device uint64 counters for stochastic calls recorded in a graph (never
// freed: they must outlive every graph that reads them).
std::mutex g_counter_mu;
std::unordered_map<int, at::Tensor>* g_counters = new std::unordered_map<int, at::Tensor>();

bool capturing() {
    return c10::hip::currentStreamCaptureStatusMayInitCtx() == c10::hip::CaptureStatus::Active;
}

at::Tensor graph_counter(int64_t index) {
    std::lock_guard<std::mutex> lk(g_counter_mu);
    auto it = g_counters->find((int)index);
    if (it != g_counters->end()) return it->second;
    c10::DeviceGuard guard(at::Device(at::kCUDA, (c10::DeviceIndex)index));
    TORCH_CHECK(!capturing(),
                "a stochastic AXS-6 call is being recorded in a HIP graph before any stochastic call ran "
                "eagerly on this device; run one warm-up step before capture (or call "
                "axs.unified.hip_kernels.prepare_graph_capture())");
    at::Tensor t = at::zeros({1}, at::TensorOptions().dtype(at::kLong).device(at::kCUDA, (c10::DeviceIndex)index));
    g_counters->emplace((int)index, t);
    return t;
}

// The capture (by its id) for which each device's counter advance has been
// recorded.  One advance per recorded graph is enough: a recorded call keys
// its dither with its own capture-time draw plus the counter, so calls that
// read the counter before and after the graph's one advance still get keys
// that differ from each other and from every other replay's, and each
// stochastic call of a graph no longer records a launch of its own.
std::unordered_map<int, unsigned long long>* g_advanced = new std::unordered_map<int, unsigned long long>();

// Records the counter's advance after a graph-recorded stochastic call on
// `device`, unless this capture already holds one.
void advance_counter(int64_t device) {
    at::Tensor c = graph_counter(device);
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    unsigned long long id = 0;
    const hipStream_t st = c10::hip::getCurrentHIPStream((c10::DeviceIndex)device).stream();
    if (hipStreamGetCaptureInfo(st, &status, &id) == hipSuccess && status == hipStreamCaptureStatusActive) {
        std::lock_guard<std::mutex> lk(g_counter_mu);
        auto it = g_advanced->find((int)device);
        if (it != g_advanced->end() && it->second == id) return;
        (*g_advanced)[(int)device] = id;
    }
    c.add_(1);
}

int64_t next_seed() {
    return at::randint(0, (int64_t)1 << 62, {1}, at::TensorOptions().dtype(at::kLong)).item<int64_t>();
}

struct Seed {
    uint64_t seed = 0;
    const uint64_t* dev = nullptr;
    at::Tensor counter;   // advanced after the call when defined
};

// The current device must be `device` (callers hold a guard).
Seed stochastic_seed(const at::Device& device, std::optional<int64_t> seed) {
    Seed s;
    s.seed = (uint64_t)(seed ? *seed : next_seed());
    if (!seed) {
        at::Tensor c = graph_counter(device.index());
        if (capturing()) {
            s.counter = c;
            s.dev = reinterpret_cast<const uint64_t*>(c.data_ptr<int64_t>());
        }
    }
    return s;
}

// ---- fake-quantize ---------------------------------------------------------------

// fused_fake_quantize (axs/unified/quantize_unified.py:121-204) on the GPU:
// blocks along the last dim, computed in the tensor's own type when it is
// float32, bfloat16 or float16 and in float32 otherwise (cast back after),
// output contiguous with the input's shape.  The caller has checked the
// device, block size and rounding mode.
at::Tensor fq(const at::Tensor& tensor, int64_t bs, bool stochastic, std::optional<int64_t> seed) {
    TORCH_CHECK_INDEX(tensor.dim() >= 1, "fake-quantize needs a tensor with a last dimension");
    const at::ScalarType orig = tensor.scalar_type();
    const at::Tensor x = (dtype_code(orig) >= 0 ? tensor : tensor.to(at::kFloat)).contiguous();
    const int64_t cols = x.size(-1);
    const int64_t rows = cols ? x.numel() / cols : 0;
    at::Tensor y = at::empty_like(x, at::MemoryFormat::Contiguous);
    if (rows && cols) {
        c10::DeviceGuard guard(x.device());
        Seed s;
        if (stochastic) s = stochastic_seed(x.device(), seed);
        check_rc(axs6_nf5_fake_quantize(x.data_ptr(), y.data_ptr(), dtype_code(x.scalar_type()), rows, cols,
                                        (int32_t)bs, stochastic ? 1 : 0, s.seed, 0, s.dev, stream_of(x)),
                 "axs6_nf5_fake_quantize");
        if (s.counter.defined()) advance_counter(x.device().index());
    }
    return y.scalar_type() == orig ? y : y.to(orig);
}

// _FusedQuantizeSTE (functional_unified.py:38-60): forward fake-quantizes,
// backward hands the incoming gradient back unchanged (the same tensor).
struct FakeQuantizeSTE : public torch::autograd::Function<FakeQuantizeSTE> {
    static at::Tensor forward(AutogradContext*, const at::Tensor& tensor, int64_t bs, bool stochastic) {
        return fq(tensor, bs, stochastic, std::nullopt);
    }
    static variable_list backward(AutogradContext*, variable_list grads) {
        return {grads[0], at::Tensor(), at::Tensor()};
    }
};

at::Tensor fq_ste(const at::Tensor& tensor, int64_t bs, bool stochastic) {
    return FakeQuantizeSTE::apply(tensor, bs, stochastic);
}

// ---- forward ------------------------------------------------------------------

struct Fwd {
    at::Tensor out, xq, sx, wq, sw;
    int64_t M, N, K, n_true, k_true;
    at::ScalarType dtype;
};

Fwd linear_fwd_impl(const at::Tensor& input, const at::Tensor& weight, const std::optional<at::Tensor>& bias,
                    int64_t bs, bool quantize_input) {
    const char* fn = "axs_linear";
    require_device(input, fn);
    require_device(weight, fn);
    TORCH_CHECK(weight.device() == input.device(), fn, ": weight is on ", weight.device(), ", input on ",
                input.device());
    TORCH_CHECK(!bias || !bias->defined() || bias->device() == input.device(), fn, ": bias is on ",
                bias && bias->defined() ? bias->device() : input.device(), ", input on ", input.device());
    TORCH_CHECK(bs == 8 || bs == 16 || bs == 32, fn, ": block_size must be one of (8, 16, 32), got ", bs);
    TORCH_CHECK(input.dim() >= 1 && weight.dim() == 2, fn, ": expected input (*, K) and weight (N, K)");
    const int64_t K = input.size(-1), N = weight.size(0), Kw = weight.size(1);
    TORCH_CHECK(Kw == K, fn, ": input has ", K, " features but weight expects ", Kw);
    const at::ScalarType dtype = compute_dtype(input.scalar_type());
    const int64_t vm = vec_multiple(dtype);
    at::Tensor x2 = dense(pad_last(rows2d(input, K).to(dtype), vm));
    at::Tensor w2 = dense(pad_rows(pad_last(weight.to(dtype), vm), vm));
    const int64_t M = x2.size(0), Kb = x2.size(1), Nb = w2.size(0);
    at::Tensor b;
    if (bias && bias->defined()) {
        b = bias_vector(*bias, N, fn).to(at::kFloat);
        if (Nb != N) b = at::constant_pad_nd(b, {0, Nb - N});
        b = b.contiguous();
    }
    const int64_t Kp = axs6_linear_padded_k(Kb);
    const auto dev = x2.options();
    Fwd r;
    r.xq = at::empty({M, Kp}, dev.dtype(at::kHalf));
    r.wq = at::empty({Nb, Kp}, dev.dtype(at::kHalf));
    r.sx = at::empty({M}, dev.dtype(at::kInt));
    r.sw = at::empty({Nb}, dev.dtype(at::kInt));
    at::Tensor y = at::empty({M, Nb}, dev.dtype(dtype));
    if (M && Nb && !Kb) {
        // an empty contraction: F.linear gives the bias (or zeros)
        if (b.defined()) y.copy_(b.to(dtype).expand({M, Nb}));
        else y.zero_();
    } else if (M && Nb) {
        c10::DeviceGuard guard(x2.device());
        check_rc(axs6_nf5_linear_forward(x2.data_ptr(), w2.data_ptr(), b.defined() ? b.data_ptr<float>() : nullptr,
                                         y.data_ptr(), dtype_code(dtype), M, Nb, Kb, (int32_t)bs,
                                         quantize_input ? 1 : 0, r.xq.data_ptr(), r.sx.data_ptr<int32_t>(),
                                         r.wq.data_ptr(), r.sw.data_ptr<int32_t>(), stream_of(x2)),
                 "axs6_nf5_linear_forward");
    }
    if (Nb != N) y = y.narrow(1, 0, N).contiguous();   // N off the vector multiple: F.linear's dense output
    r.out = to_input_dtype(y.reshape(lead_shape(input.sizes(), N)), input.scalar_type());
    r.M = M; r.N = Nb; r.K = Kb; r.n_true = N; r.k_true = K; r.dtype = dtype;
    return r;
}

// ---- backward -----------------------------------------------------------------

std::tuple<at::Tensor, at::Tensor, at::Tensor> linear_bwd_impl(
    const at::Tensor& grad_output, const at::Tensor& xq, const at::Tensor& sx, const at::Tensor& wq,
    const at::Tensor& sw, int64_t M, int64_t N, int64_t K, int64_t n_true, int64_t k_true, at::ScalarType dtype,
    at::IntArrayRef x_shape, at::ScalarType w_dtype, int64_t bs, bool quantize_grad, bool need_x, bool need_w,
    bool need_b, std::optional<int64_t> seed, std::optional<at::ScalarType> x_dtype) {
    const auto opts = xq.options();
    TORCH_CHECK(grad_output.device() == xq.device(), "axs_linear backward: grad_output is on ", grad_output.device(),
                ", the saved operands on ", xq.device());
    TORCH_CHECK(grad_output.numel() == M * n_true, "axs_linear backward: grad_output has ", grad_output.numel(),
                " elements, expected ", M * n_true);
    at::Tensor dy = rows2d(grad_output, n_true).to(dtype);
    if (N != n_true) dy = pad_last(dy, vec_multiple(dtype));
    dy = dense(dy);
    at::Tensor dx, dw, db;
    if (need_x) dx = at::empty({M, K}, opts.dtype(dtype));
    if (need_w) dw = at::empty({N, K}, opts.dtype(at::kFloat));
    if (need_b) db = at::empty({N}, opts.dtype(at::kFloat));
    if (M && N && (need_x || need_w || need_b)) {
        c10::DeviceGuard guard(dy.device());
        const size_t ws_bytes = axs6_nf5_linear_backward_workspace(M, N, K, need_x, need_w, need_b);
        at::Tensor ws = at::empty({(int64_t)ws_bytes}, opts.dtype(at::kByte));
        Seed s;
        if (quantize_grad) s = stochastic_seed(dy.device(), seed);
        check_rc(axs6_nf5_linear_backward(
                     dy.data_ptr(), dtype_code(dtype), M, N, K, (int32_t)bs, quantize_grad ? 1 : 0, s.seed, 0,
                     xq.data_ptr(), sx.data_ptr<int32_t>(), wq.data_ptr(), sw.data_ptr<int32_t>(),
                     need_x ? dx.data_ptr() : nullptr, need_w ? dw.data_ptr<float>() : nullptr,
                     need_b ? db.data_ptr<float>() : nullptr, ws.data_ptr(), ws_bytes, s.dev, stream_of(dy)),
                 "axs6_nf5_linear_backward");
        if (s.counter.defined()) advance_counter(dy.device().index());
    } else {
        // no rows (M == 0): the reference's dYq^T X and sum over rows give zeros
        if (dw.defined()) dw.zero_();
        if (db.defined()) db.zero_();
    }
    if (dx.defined()) {
        if (K != k_true) dx = dx.narrow(1, 0, k_true);
        dx = dx.reshape(lead_shape(x_shape, k_true));
        if (x_dtype) dx = to_input_dtype(dx, *x_dtype);
    }
    if (dw.defined()) {
        dw = dw.narrow(0, 0, n_true).narrow(1, 0, k_true);
        if (w_dtype != at::kFloat) dw = dw.to(w_dtype);
    }
    if (db.defined()) db = db.narrow(0, 0, n_true);
    return {dx, dw, db};
}

// ---- autograd node --------------------------------------------------------------

struct LinearFunction : public torch::autograd::Function<LinearFunction> {
    static at::Tensor forward(AutogradContext* ctx, const at::Tensor& input, const at::Tensor& weight,
                              const at::Tensor& bias, int64_t bs, bool quantize_input, bool quantize_grad,
                              bool has_bias) {
        Fwd r = linear_fwd_impl(input, weight, has_bias ? std::optional<at::Tensor>(bias) : std::nullopt, bs,
                                quantize_input);
        ctx->save_for_backward({r.xq, r.sx, r.wq, r.sw});
        auto& d = ctx->saved_data;
        d["M"] = r.M; d["N"] = r.N; d["K"] = r.K; d["n_true"] = r.n_true; d["k_true"] = r.k_true;
        d["dtype"] = (int64_t)r.dtype;
        d["w_dtype"] = (int64_t)weight.scalar_type();
        d["x_dtype"] = (int64_t)input.scalar_type();
        d["x_shape"] = input.sizes().vec();
        d["bs"] = bs;
        d["quantize_grad"] = quantize_grad;
        d["has_bias"] = has_bias;
        return r.out;
    }

    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        const at::Tensor& g = grads[0];
        if (!g.defined())
            return {at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor()};
        const auto saved = ctx->get_saved_variables();
        auto& d = ctx->saved_data;
        const bool need_x = ctx->needs_input_grad(0), need_w = ctx->needs_input_grad(1);
        const bool need_b = ctx->needs_input_grad(2) && d["has_bias"].toBool();
        const auto x_shape = d["x_shape"].toIntVector();
        auto [dx, dw, db] = linear_bwd_impl(
            g, saved[0], saved[1], saved[2], saved[3], d["M"].toInt(), d["N"].toInt(), d["K"].toInt(),
            d["n_true"].toInt(), d["k_true"].toInt(), (at::ScalarType)d["dtype"].toInt(), x_shape,
            (at::ScalarType)d["w_dtype"].toInt(), d["bs"].toInt(), d["quantize_grad"].toBool(), need_x, need_w,
            need_b, std::nullopt, (at::ScalarType)d["x_dtype"].toInt());
        return {dx, dw, db, at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor()};
    }
};

at::Tensor linear(const at::Tensor& input, const at::Tensor& weight, const std::optional<at::Tensor>& bias,
                  int64_t bs, bool quantize_input, bool quantize_grad) {
    // the autograd node records every tensor argument's device, so a missing
    // bias travels as an empty tensor (no storage) that forward() treats as absent
    const bool has_bias = bias && bias->defined();
    return LinearFunction::apply(input, weight, has_bias ? *bias : at::empty({0}, input.options()), bs,
                                 quantize_input, quantize_grad, has_bias);
}

py::tuple linear_fwd(const at::Tensor& input, const at::Tensor& weight, const std::optional<at::Tensor>& bias,
                     int64_t bs, bool quantize_input) {
    Fwd r = linear_fwd_impl(input, weight, bias, bs, quantize_input);
    return py::make_tuple(r.out, r.xq, r.sx, r.wq, r.sw, r.M, r.N, r.K, r.n_true, r.k_true, r.dtype);
}

// ---- LayerNorm (AXSLayerNormUnified) ---------------------------------------------

// F.layer_norm over the last `ndim` dims (modules_unified.py:141-144) as one
// autograd node over axs6_layer_norm_forward / _backward: float32, bfloat16
// or float16 input with weight and bias of the same dtype (or absent).
struct LayerNormFunction : public torch::autograd::Function<LayerNormFunction> {
    static at::Tensor forward(AutogradContext* ctx, const at::Tensor& input, const at::Tensor& weight,
                              const at::Tensor& bias, int64_t ndim, double eps, bool has_weight, bool has_bias) {
        const char* fn = "axs6_layer_norm_forward";
        require_device(input, fn);
        const int dt = dtype_code(input.scalar_type());
        TORCH_CHECK(dt >= 0, "layer_norm: input dtype ", input.scalar_type(), " is not float32, bfloat16 or float16");
        TORCH_CHECK(ndim >= 1 && ndim <= input.dim(), "layer_norm: normalized_shape of ", ndim,
                    " dims for an input of ", input.dim());
        int64_t cols = 1;
        for (int64_t d = input.dim() - ndim; d < input.dim(); ++d) cols *= input.size(d);
        const int64_t rows = cols ? input.numel() / cols : 0;
        for (const at::Tensor* p : {&weight, &bias}) {
            if ((p == &weight && !has_weight) || (p == &bias && !has_bias)) continue;
            TORCH_CHECK(p->device() == input.device() && p->scalar_type() == input.scalar_type() &&
                            p->numel() == cols,
                        "layer_norm: weight and bias must be ", cols, " values of the input's dtype and device");
        }
        c10::DeviceGuard guard(input.device());
        at::Tensor x = input.contiguous();
        at::Tensor w = has_weight ? weight.contiguous() : at::Tensor();
        at::Tensor b = has_bias ? bias.contiguous() : at::Tensor();
        at::Tensor y = at::empty_like(x);
        at::Tensor mean = at::empty({rows}, x.options().dtype(at::kFloat));
        at::Tensor rstd = at::empty({rows}, x.options().dtype(at::kFloat));
        check_rc(axs6_layer_norm_forward(x.data_ptr(), dt, rows, cols, has_weight ? w.data_ptr() : nullptr,
                                         has_bias ? b.data_ptr() : nullptr, (float)eps, y.data_ptr(),
                                         mean.data_ptr<float>(), rstd.data_ptr<float>(), stream_of(x)),
                 fn);
        ctx->save_for_backward({x, has_weight ? w : at::Tensor(), mean, rstd});
        auto& d = ctx->saved_data;
        d["rows"] = rows; d["cols"] = cols; d["has_weight"] = has_weight; d["has_bias"] = has_bias;
        d["nshape"] = input.sizes().slice(input.dim() - ndim).vec();
        return y;
    }

    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        const char* fn = "axs6_layer_norm_backward";
        variable_list none(7);
        if (!grads[0].defined()) return none;
        const auto saved = ctx->get_saved_variables();
        const at::Tensor& x = saved[0];
        auto& d = ctx->saved_data;
        const int64_t rows = d["rows"].toInt(), cols = d["cols"].toInt();
        const bool has_w = d["has_weight"].toBool(), has_b = d["has_bias"].toBool();
        const bool need_w = has_w && ctx->needs_input_grad(1), need_b = has_b && ctx->needs_input_grad(2);
        c10::DeviceGuard guard(x.device());
        at::Tensor dy = grads[0].to(x.scalar_type()).contiguous();
        at::Tensor dx = at::empty_like(x);
        const auto f32 = x.options().dtype(at::kFloat);
        at::Tensor dw = need_w ? at::empty({cols}, f32) : at::Tensor();
        at::Tensor db = need_b ? at::empty({cols}, f32) : at::Tensor();
        const int64_t ws = axs6_layer_norm_backward_workspace(rows, cols);
        TORCH_CHECK(ws >= 0, fn, ": bad shape");
        at::Tensor work = at::empty({ws > 0 ? ws : 1}, x.options().dtype(at::kByte));
        check_rc(axs6_layer_norm_backward(dy.data_ptr(), x.data_ptr(), dtype_code(x.scalar_type()), rows, cols,
                                          saved[2].data_ptr<float>(), saved[3].data_ptr<float>(),
                                          has_w ? saved[1].data_ptr() : nullptr, dx.data_ptr(),
                                          need_w ? dw.data_ptr<float>() : nullptr,
                                          need_b ? db.data_ptr<float>() : nullptr, work.data_ptr(), (size_t)ws,
                                          stream_of(x)),
                 fn);
        variable_list out(7);
        out[0] = dx;
        const auto nshape = d["nshape"].toIntVector();
        if (need_w) out[1] = dw.to(x.scalar_type()).view(nshape);
        if (need_b) out[2] = db.to(x.scalar_type()).view(nshape);
        return out;
    }
};

at::Tensor layer_norm(const at::Tensor& input, const std::optional<at::Tensor>& weight,
                      const std::optional<at::Tensor>& bias, int64_t ndim, double eps) {
    // absent parameters travel as empty tensors (see linear())
    const bool hw = weight && weight->defined(), hb = bias && bias->defined();
    const at::Tensor empty = at::empty({0}, input.options());
    return LayerNormFunction::apply(input, hw ? *weight : empty, hb ? *bias : empty, ndim, eps, hw, hb);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "AXS-6 fake-quantize and quantized linear: host logic and autograd nodes over libaxs6.so";
    m.def("fq", &fq, "NF5 fake-quantize of the last dim (no autograd)", py::arg("tensor"), py::arg("block_size"),
          py::arg("stochastic"), py::arg("seed") = py::none());
    m.def("fq_ste", &fq_ste, "NF5 fake-quantize with the straight-through gradient (autograd node)",
          py::arg("tensor"), py::arg("block_size"), py::arg("stochastic"));
    m.def("layer_norm", &layer_norm,
          "F.layer_norm over the last `ndim` dims on the HIP kernels (autograd node)", py::arg("input"),
          py::arg("weight"), py::arg("bias"), py::arg("ndim"), py::arg("eps"));
    m.def("linear", &linear, "FQ(input) FQ(weight)^T + bias with the quantized backward (autograd node)",
          py::arg("input"), py::arg("weight"), py::arg("bias"), py::arg("block_size"), py::arg("quantize_input"),
          py::arg("quantize_grad"));
    m.def("linear_fwd", &linear_fwd,
          "forward: (out, xq, sx, wq, sw, M, N, K, n_true, k_true, dtype) -- packed operands for the backward",
          py::arg("input"), py::arg("weight"), py::arg("bias"), py::arg("block_size"), py::arg("quantize_input"));
    m.def("linear_bwd", &linear_bwd_impl, "backward: (dx, dw, db), each None when not requested",
          py::arg("grad_output"), py::arg("xq"), py::arg("sx"), py::arg("wq"), py::arg("sw"), py::arg("M"),
          py::arg("N"), py::arg("K"), py::arg("n_true"), py::arg("k_true"), py::arg("dtype"), py::arg("x_shape"),
          py::arg("w_dtype"), py::arg("block_size"), py::arg("quantize_grad"), py::arg("need_x"), py::arg("need_w"),
          py::arg("need_b"), py::arg("seed") = py::none(), py::arg("x_dtype") = py::none());
    m.def("graph_counter", &graph_counter, "the device's dither counter for graph-recorded stochastic calls",
          py::arg("index"));
    m.def("graph_counter_advance", &advance_counter,
          "records the device's counter advance after a graph-recorded stochastic call (once per capture)",
          py::arg("device"));
    m.def("next_seed", &next_seed, "a dither seed from torch's default CPU generator");
}
