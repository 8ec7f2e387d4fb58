// TEST INFRASTRUCTURE: a C-ABI wrapper around the reference's own
// sources/scalar_math.h (exponential, silu, gelu), compiled unmodified from
// where it lies under the reference checkout (ref.mk), into oracle/_ref/.  The
// tests hold the oracle's restatement (oracle.c) and the device's functions
// (csrc/device.h, through the library) to these bits.  Nothing of the library
// links it.
#include <cstdint>

#include "scalar_math.h"

extern "C" {

float ref_exponential(float x) { return sdasm::exponential(x); }
float ref_silu(float x) { return sdasm::silu(x); }
float ref_gelu(float x) { return sdasm::gelu(x); }

void ref_exponential_array(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = sdasm::exponential(x[i]);
}
void ref_silu_array(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = sdasm::silu(x[i]);
}
void ref_gelu_array(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = sdasm::gelu(x[i]);
}

}  // extern "C"
