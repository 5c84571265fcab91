// Internal declarations shared by the libaxs6 translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "axs6.h"

namespace axs6 {

constexpr int kLevels = 32;
constexpr int kLutSize = 1024;
constexpr int kLutMax = 1023;
constexpr int kBandSize = 288;   // band[k + 149] for k in [-148, 128]; padded to 72 words
constexpr int kExpBias = 127;

// Device copies of the constant tables, one set per device.
struct DeviceTables {
    const float* codebook;   // 32
    const float* lut;        // 1024
    const uint8_t* rev;      // 1024
    const uint8_t* band;     // kBandSize
};

// Host tables (built once, process-wide).
void host_tables(float* codebook, float* lut, uint8_t* rev, uint8_t* band);

// Uploads tables to the current device on first use; fills *out.
int device_tables(DeviceTables* out);

// Resolves the current device's address of the allocation-free backward's
// scratch array (nf5_linear.hip); called by axs6_init.
int init_noalloc_scratch();

// Records a message for axs6_last_error() and returns `code`.
int fail(int code, const char* fmt, ...);

// Checks the last launch on this thread.
int check_launch(const char* what);

inline bool valid_block(int bs) { return bs == 8 || bs == 16 || bs == 32; }
inline bool valid_dtype(int dt) { return dt == AXS6_F32 || dt == AXS6_BF16 || dt == AXS6_F16; }

}  // namespace axs6
