// libaxs6 runtime: constant tables, per-device upload, error reporting.
//
// The tables are the NF5 format's constants:
//   codebook  32 half-normal quantile levels, cb[i] = sqrt2*erfinv((i+0.5)/32)
//             normalised by cb[31] and rounded to float32 -- the values of
//             NF5_CODEBOOK (axs/unified/quantize_unified.py:50-61), stored
//             here as their float32 bit patterns;
//   lut       1024-entry fused LUT: lut[i] = cb[code(i/1023)], code from the
//             float64 midpoints (axs/unified/quantize_unified.py:68-97);
//   rev       LUT index -> code (axs/unified/quantize_unified.py:105-114);
//   band      log2 rounding band: torch's CPU float32 log2 is correctly
//             rounded, so floor(log2(x)) equals k for the band[k+149] float32
//             values just below 2^k (e.g. 44 of them below 2^127).  The
//             kernels take floor(log2(amax)) from the exponent bits and add
//             one inside the band, which reproduces
//             floor(torch.log2(amax)) (quantize_unified.py:173-175) exactly.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "axs6_internal.h"

namespace axs6 {

namespace {

constexpr uint32_t kCodebookBits[kLevels] = {
    0x3c04b96eu, 0x3cc7303eu, 0x3d26292au, 0x3d68fc26u, 0x3d96163bu, 0x3db7eb43u,
    0x3dda0c14u, 0x3dfc887bu, 0x3e0fb8b1u, 0x3e216c8au, 0x3e3369c5u, 0x3e45bb68u,
    0x3e586dbbu, 0x3e6b8e8eu, 0x3e7f2d9bu, 0x3e89ae7au, 0x3e9418d0u, 0x3e9ee22eu,
    0x3eaa1958u, 0x3eb5d02bu, 0x3ec21ca7u, 0x3ecf1a59u, 0x3edcec91u, 0x3eebc1b0u,
    0x3efbd888u, 0x3f06c4beu, 0x3f10ab83u, 0x3f1c0741u, 0x3f2988aeu, 0x3f3a8bf4u,
    0x3f5273dcu, 0x3f800000u};

struct HostTables {
    float codebook[kLevels];
    float lut[kLutSize];
    uint8_t rev[kLutSize];
    uint8_t band[kBandSize];
};

float bits_to_float(uint32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}

uint32_t float_to_bits(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    return b;
}

HostTables build_host_tables() {
    HostTables t;
    memset(&t, 0, sizeof t);
    for (int i = 0; i < kLevels; ++i) t.codebook[i] = bits_to_float(kCodebookBits[i]);

    // Fused LUT: code(x) = #{boundaries < x} - 1 with boundaries
    // [0, midpoints (float64), 1 + 1e-6], x = linspace(0, 1, 1024) in float64
    // (first half counted up from 0, second half down from 1).
    double bnd[kLevels + 1];
    bnd[0] = 0.0;
    for (int i = 0; i + 1 < kLevels; ++i)
        bnd[i + 1] = ((double)t.codebook[i] + (double)t.codebook[i + 1]) / 2.0;
    bnd[kLevels] = 1.0 + 1e-6;
    const double step = 1.0 / (double)(kLutSize - 1);
    for (int i = 0; i < kLutSize; ++i) {
        double x = (i < kLutSize / 2) ? step * (double)i : 1.0 - step * (double)(kLutSize - 1 - i);
        int below = 0;
        for (int j = 0; j <= kLevels; ++j) below += (bnd[j] < x) ? 1 : 0;
        int code = below - 1;
        code = code < 0 ? 0 : (code > kLevels - 1 ? kLevels - 1 : code);
        t.lut[i] = t.codebook[code];
        t.rev[i] = (uint8_t)code;
    }

    // log2 band: for each k, count float32 values x just below 2^k whose
    // correctly rounded float32 log2 equals k.  long double log2l carries
    // 64 mantissa bits, far more than the float32 rounding decision needs.
    for (int k = -148; k <= 128; ++k) {
        uint32_t top = (k >= -126) ? (uint32_t)(k + 127) << 23 : (1u << (k + 149));
        int count = 0;
        for (int m = 1; m < 255; ++m) {
            if ((uint32_t)m >= top) break;
            float x = bits_to_float(top - (uint32_t)m);
            float l = (float)log2l((long double)x);
            if (l == (float)k) ++count;
            else break;
        }
        t.band[k + 149] = (uint8_t)count;
    }
    return t;
}

const HostTables& tables() {
    static const HostTables t = build_host_tables();
    return t;
}

// Device-resident copies: one instance of each array per device, filled by
// hipMemcpyToSymbol with that device current; kernels in every translation
// unit receive their addresses (hipGetSymbolAddress) as arguments.
__device__ float d_codebook[kLevels];
__device__ float d_lut[kLutSize];
__device__ uint8_t d_rev[kLutSize];
__device__ uint8_t d_band[kBandSize];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
bool g_ready[kMaxDevices];
DeviceTables g_dev[kMaxDevices];

thread_local char g_err[512];

}  // namespace

void host_tables(float* codebook, float* lut, uint8_t* rev, uint8_t* band) {
    const HostTables& t = tables();
    if (codebook) memcpy(codebook, t.codebook, sizeof t.codebook);
    if (lut) memcpy(lut, t.lut, sizeof t.lut);
    if (rev) memcpy(rev, t.rev, sizeof t.rev);
    if (band) memcpy(band, t.band, 278);
}

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(AXS6_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return AXS6_OK;
}

int device_tables(DeviceTables* out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0) return fail(AXS6_ERR_NO_DEVICE, "no current HIP device: %s", hipGetErrorString(e));
    if (dev >= kMaxDevices) return fail(AXS6_ERR_UNSUPPORTED, "device ordinal %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ready[dev]) {
        const HostTables& t = tables();
        if ((e = hipMemcpyToSymbol(HIP_SYMBOL(d_codebook), t.codebook, sizeof t.codebook)) != hipSuccess ||
            (e = hipMemcpyToSymbol(HIP_SYMBOL(d_lut), t.lut, sizeof t.lut)) != hipSuccess ||
            (e = hipMemcpyToSymbol(HIP_SYMBOL(d_rev), t.rev, sizeof t.rev)) != hipSuccess ||
            (e = hipMemcpyToSymbol(HIP_SYMBOL(d_band), t.band, sizeof t.band)) != hipSuccess)
            return fail(AXS6_ERR_HIP, "table upload to device %d failed: %s", dev, hipGetErrorString(e));
        void *p0, *p1, *p2, *p3;
        if ((e = hipGetSymbolAddress(&p0, HIP_SYMBOL(d_codebook))) != hipSuccess ||
            (e = hipGetSymbolAddress(&p1, HIP_SYMBOL(d_lut))) != hipSuccess ||
            (e = hipGetSymbolAddress(&p2, HIP_SYMBOL(d_rev))) != hipSuccess ||
            (e = hipGetSymbolAddress(&p3, HIP_SYMBOL(d_band))) != hipSuccess)
            return fail(AXS6_ERR_HIP, "table address lookup on device %d failed: %s", dev, hipGetErrorString(e));
        g_dev[dev] = DeviceTables{(const float*)p0, (const float*)p1, (const uint8_t*)p2, (const uint8_t*)p3};
        g_ready[dev] = true;
    }
    *out = g_dev[dev];
    return AXS6_OK;
}

}  // namespace axs6

extern "C" {

const char* axs6_version(void) { return "axs6-mi355x 0.1.0 (gfx950)"; }

const char* axs6_last_error(void) { return axs6::g_err; }

int axs6_init(void) {
    axs6::g_err[0] = 0;
    axs6::DeviceTables t;
    int rc = axs6::device_tables(&t);
    return rc ? rc : axs6::init_noalloc_scratch();
}

int axs6_get_tables(float* codebook, float* lut, uint8_t* reverse_lut, uint8_t* log2_band) {
    axs6::host_tables(codebook, lut, reverse_lut, log2_band);
    return AXS6_OK;
}

}  // extern "C"
