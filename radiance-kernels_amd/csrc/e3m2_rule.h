// The R1 E3M2 element rule on 32-bit patterns (lib/golden/mx_fp_math.h:11-28, 266-335: bf16 RNE,
// then the E4M2 rounding and the fixed E4M2 -> E3M2 value map), and its branch-free table form
// used by the quantizers.  Plain C++ on integers (bit casts, no device builtins), so that the
// same source also builds for the host: tests/test_e3m2_table.py compiles it with g++ and
// checks the table form against the rule on all 2^32 floats.
#pragma once

#include <stdint.h>

namespace mxfa {

// lib/golden bf16 RNE (+-0 -> +0, tiny -> +0, NaN quieted).
__device__ __forceinline__ uint32_t bf16_rne(float x) {
  if (x == 0.0f) return 0u;
  uint32_t b = __builtin_bit_cast(uint32_t, x);
  if (((b >> 23) & 0xffu) == 0xffu) {
    uint32_t h = b >> 16;
    if ((b & 0x7fffffu) && !(h & 0x40u)) h |= 0x40u;
    return h & 0xffffu;
  }
  uint32_t r = (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
  return (r & 0x7fffu) == 0u ? 0u : r;
}

// R1 E3M2 code (6 bits, one per byte) of a bf16 pattern.
__device__ __forceinline__ uint32_t e3m2_code_bf16(uint32_t h) {
  uint32_t neg = (h >> 15) & 1u;
  int E = (int)((h >> 7) & 0xffu), M = (int)(h & 0x7fu);
  if (E == 0) return 0u;
  uint32_t c;
  if (E == 255) {
    c = 0x1fu;                                   // inf / NaN -> E4M2 inf -> +-28
  } else {
    int e = E - 127;
    if (e > 7 || e < -6) return 0u;              // reference maps both tails to 0
    int q = M >> 5, r = (M >> 4) & 1, st = (M & 15) != 0;
    int sig = q + (r & (st | (q & 1)));
    if (sig == 4) { sig = 0; e++; }
    if (e >= 5) c = 0x1fu;                       // >= 32 (or E4M2 overflow) -> 28
    else if (e >= -2) c = ((uint32_t)(e + 3) << 2) | (uint32_t)sig;
    else if (e == -3) c = sig < 2 ? 2u : 3u;     // 0.125 / 0.1875
    else if (e == -4) c = sig < 2 ? 1u : 2u;     // 0.0625 / 0.125
    else return 0u;                              // <= 0.0546875
  }
  return (neg << 5) | c;
}

// E3M2 codes through a table.  e3m2_code_bf16 gives non-zero finite codes only for bf16
// exponent fields 121 .. 134; the table holds its value for those 14 x 128 magnitudes, filled
// per workgroup from e3m2_code_bf16 itself (e3m2_tab_fill), and e3m2_code_tab(y, tab) equals
// e3m2_code_bf16(bf16_rne(y)) for every float y, branch-free: |y| rounded to bf16 by integer
// add and shift, the table for the 14 binades, 0 below and above them, 28 (0x1f) for
// magnitudes that round to inf and for inf / NaN, the sign on non-zero codes.
constexpr int E3M2_TAB_E0 = 121, E3M2_TAB_N = 14 * 128;

__device__ __forceinline__ void e3m2_tab_fill(uint8_t* tab, int tid, int nthreads) {
  for (int i = tid; i < E3M2_TAB_N; i += nthreads) tab[i] = (uint8_t)e3m2_code_bf16((uint32_t)((E3M2_TAB_E0 << 7) + i));
}

__device__ __forceinline__ uint32_t e3m2_code_tab(float y, const uint8_t* tab) {
  const uint32_t b = __builtin_bit_cast(uint32_t, y), a = b & 0x7fffffffu;
  const uint32_t mag = (a + 0x7fffu + ((a >> 16) & 1u)) >> 16;     // bf16 RNE of |y| (>= 0x7f80: inf / NaN)
  const uint32_t idx = mag - (uint32_t)(E3M2_TAB_E0 << 7);
  const bool in = idx < (uint32_t)E3M2_TAB_N;
  const uint32_t t = tab[in ? idx : 0u];
  const uint32_t c = mag >= 0x7f80u ? 0x1fu : in ? t : 0u;
  return c ? c | ((b >> 26) & 0x20u) : 0u;
}

}  // namespace mxfa
