// Thin extern "C" wrapper that exposes the reference's own lib/golden MX
// element rules (compiled from /root/reference/lib/golden/mx_fp_math.h where
// it lies; nothing of it is copied here) to the oracle's tests.  Built only
// into oracle/_ref/ by oracle/Makefile, never shipped with the product.
#include <cstdint>
#include <cstring>
#include "mx_fp_math.h"

extern "C" {
// Encode count float bit patterns starting at bits_lo with fp8_e4m3_to_code.
void ref_e4m3_encode_range(uint32_t bits_lo, uint32_t count, uint8_t *out) {
  for (uint32_t i = 0; i < count; i++) {
    uint32_t b = bits_lo + i;
    float f;
    std::memcpy(&f, &b, 4);
    out[i] = mx::fp8_e4m3_to_code(f);
  }
}
void ref_e4m3_encode_array(const float *x, int64_t n, uint8_t *out) {
  for (int64_t i = 0; i < n; i++) out[i] = mx::fp8_e4m3_to_code(x[i]);
}
float ref_e4m3_decode(uint8_t c) { return mx::fp8_e4m3_decode(c); }
float ref_e3m2_decode(uint8_t c) { return mx::fp6_e3m2_decode(c); }
float ref_e8m0_decode(uint8_t c) { return mx::fpe8m0_decode(c); }
uint8_t ref_e3m2_encode_bf16(uint16_t b) { return mx::bf16_bits_to_fp6_e3m2_code(b); }
void ref_f32_to_bf16_array(const float *x, int64_t n, uint16_t *out) {
  for (int64_t i = 0; i < n; i++) out[i] = mx::f32_to_bf16_rne(x[i]);
}
}
