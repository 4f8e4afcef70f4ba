// Device-side MX rules for gfx950 (CDNA4).
//
// Rule "R1" of the reference's lib/golden C code, bit-exact:
//   block scale  : code = clamp(floor(log2f(amax)) - P + 127, 0, 254), P = 8 (E4M3)
//                  or 4 (E3M2), amax == 0 -> 0        (lib/golden/mx_golden.cpp:169-174)
//   E4M3 element : floor(log2f(|y|)) < -6 -> 0, > 8 -> +-448, else RNE to 3 mantissa
//                  bits, saturating at 448           (lib/golden/mx_fp_math.h:205-225)
//   E3M2 element : bf16 RNE, then RNE to E4M2, then the fixed E4M2 -> E3M2 value
//                  map                                (lib/golden/mx_fp_math.h:11-28, 266-335)
// floorf(log2f(x)) is reproduced from the exponent plus a per-binade mantissa
// threshold (log2f rounds to float, so values just below 2^(e+1) give e+1).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "e3m2_rule.h"
#include "log2_table.h"

namespace mxfa {

__constant__ uint32_t c_log2_thr[256] = MXFA_LOG2_THR_INIT;
__constant__ uint32_t c_log2_sub_thr[23] = MXFA_LOG2_SUB_THR_INIT;

// floorf(log2f(x)) for finite x > 0 (x == 0 returns a large negative number).
__device__ __forceinline__ int floor_log2f(float x) {
  uint32_t b = __float_as_uint(x) & 0x7fffffffu;
  uint32_t E = b >> 23, m = b & 0x7fffffu;
  if (E == 0) {
    if (m == 0) return -1024;
    int p = 31 - __clz(m);
    return p - 149 + (m >= c_log2_sub_thr[p] ? 1 : 0);
  }
  return (int)E - 127 + (m >= c_log2_thr[E] ? 1 : 0);
}

// E8M0 block scale code; amax = max |x| over the block (NaN already dropped by fmaxf).
__device__ __forceinline__ uint32_t scale_code(float amax, int log2_pmax) {
  if (!(amax > 0.0f) || __builtin_isinf(amax)) return 0u;
  int s2 = floor_log2f(amax) - log2_pmax + 127;
  return (uint32_t)(s2 < 0 ? 0 : (s2 > 254 ? 254 : s2));
}

// E4M3 block scale code of a finite amax >= 0 (the P blocks), without a table or
// branches.  For a normal amax with exponent e, floorf(log2f(amax)) is e + 1 when the
// mantissa reaches 2^23 - delta, where delta depends only on the binade of
// u = (e >= 0 ? e : -e - 1) (log2f rounds to the float grid around e + 1).  An amax
// below 2^-119 (zero and subnormals included) gives floor - 8 + 127 < 0, i.e. code 0,
// and a finite amax stays below the 254 clamp.
__device__ __forceinline__ uint32_t scale_code_p(float amax) {
  uint32_t b = __float_as_uint(amax);
  int e = (int)(b >> 23) - 127;
  uint32_t u = (uint32_t)(e ^ (e >> 31));            // e >= 0 ? e : -e - 1
  int k = 31 - __clz(u | 1u);
  uint32_t delta = (uint32_t)((0x2C160B05020100ull >> (8 * k)) & 0xffu);
  uint32_t thr = u < 2u ? 0x800000u : 0x800000u - delta;
  int s = e + 119 + ((b & 0x7fffffu) >= thr ? 1 : 0);
  return s < 0 ? 0u : (uint32_t)s;
}

// The same code with a fast path for the attention P tiles: the round-up term of
// scale_code_p (floorf(log2f()) = e + 1) needs a mantissa of at least 2^23 - 0x2c, so when
// no lane of the wave has one the code is max(exponent field - 8, 0); otherwise the whole
// wave takes the closed form.  Wave-uniform branch; the result equals scale_code_p.
__device__ __forceinline__ uint32_t scale_code_p_fast(float amax) {
  const uint32_t b = __float_as_uint(amax);
  const int s = (int)(b >> 23) - 8;
  uint32_t sc = (uint32_t)(s < 0 ? 0 : s);
  if (__builtin_expect(__any((b & 0x7fffffu) >= 0x7fffd4u), 0)) {
    __asm__ volatile("");          // keeps the closed form behind the branch
    sc = scale_code_p(amax);
  }
  return sc;
}

// The same code without a branch, for a tile amax in [0, 1] (every P tile: amax =
// exp2((tile max - row max) * c) with tile max <= row max).  floorf(log2f(amax)) is e + 1
// instead of e when the mantissa lies within delta of 2^23, where delta depends on the
// binade's distance below 2^0, u = 126 - E: delta = 0x2C >> (6 - floor(log2 u)) for
// u >= 2 (the 0x01, 0x02, 0x05, 0x0B, 0x16, 0x2C of scale_code_p) and 0 below.  Adding
// delta to the bit pattern carries into the exponent field exactly when the mantissa
// reaches 2^23 - delta, so the code is max(((bits + delta) >> 23) - 8, 0).  Equal to
// scale_code_p for every float in [0, 1] (checked exhaustively).
__device__ __forceinline__ uint32_t scale_code_p_nb(float amax) {
  const uint32_t b = __float_as_uint(amax);
  const uint32_t u = __builtin_elementwise_sub_sat(126u, b >> 23);   // 126 - E, 0 at E = 127
  const uint32_t delta = 0x58000000u >> __builtin_clz(u | 1u);
  return __builtin_elementwise_sub_sat((b + delta) >> 23, 8u);
}

// Rule R4, the reference's SIMT block quantizer (kernels/simt_quant/kernel.cpp:43-117):
// E4M3 code of y with round-half-even, saturation at 448 and subnormals kept (2^-9 grid).
__device__ __forceinline__ uint32_t r4_round_shift(uint32_t v, int sh) {   // RNE of v / 2^sh, sh > 0
  if (sh >= 32) return 0u;
  const uint32_t low = v & ((1u << sh) - 1u), half = 1u << (sh - 1), q = v >> sh;
  return q + ((low > half || (low == half && (q & 1u))) ? 1u : 0u);
}

__device__ __forceinline__ uint32_t r4_e4m3_code(float y) {
  const uint32_t x = __float_as_uint(y), s = ((x >> 31) & 1u) << 7, a = x & 0x7fffffffu;
  if (a == 0u) return s;
  if (__uint_as_float(a) >= 448.0f) return s | 0x7eu;
  const int e = (int)((a >> 23) & 0xffu) - 127;
  const uint32_t sig = (1u << 23) | (a & 0x7fffffu);
  if (e < -6) {
    const uint32_t q = r4_round_shift(sig, 14 - e);
    return s | (q >= 8u ? (8u | (q - 8u)) : q);
  }
  uint32_t r = r4_round_shift(sig, 20);
  int E = e;
  if (r == 16u) { r = 8u; E++; }
  const int ef = E + 7;
  const uint32_t m = r - 8u;
  if (ef > 15 || (ef == 15 && m == 7u)) return s | 0x7eu;
  return s | ((uint32_t)ef << 3) | m;
}

// R4 block scale from amax's bits: e = ceil(log2(amax / 448)) = (E - 135) + (mantissa >
// 0x600000); code clamp(e + 127, 0, 254); the element multiplier 2^-e is built from the
// 32-bit word (127 - e) << 23 exactly as the reference builds it.  amax == 0: code 0, 1.
__device__ __forceinline__ uint32_t r4_scale(float amax, float& mul) {
  if (amax == 0.0f) {
    mul = 1.0f;
    return 0u;
  }
  const uint32_t ab = __float_as_uint(amax);
  const int e = ((int)((ab >> 23) & 0xffu) - 135) + ((ab & 0x7fffffu) > 0x600000u ? 1 : 0);
  mul = __uint_as_float((uint32_t)(127 - e) << 23);
  const int c = e + 127;
  return (uint32_t)(c < 0 ? 0 : (c > 254 ? 254 : c));
}



// Element i (a 6-bit code) of a 32-element block packed little endian into six dwords: bits
// 6i .. 6i + 5 of the 192 (i a compile-time constant after unrolling).
// Field of row r (0..31) in a block-packed E3M2 block: rows 8g + 4a + b (g < 4, a < 2, b < 4)
// at field 16a + 4g + b.  The attention kernels' P operand holds, in lane half a, byte 4g +
// b of each 16-byte half t, the probability of key 32t + 8g + 4a + b; the scaled MFMA pairs
// that byte with fp6 A field 16a + 4g + b of lane half t, so V stored in this order is read
// with the key order P has.
__device__ __forceinline__ constexpr int blk6_field(int r) { return 16 * ((r >> 2) & 1) + 4 * (r >> 3) + (r & 3); }

__device__ __forceinline__ void pack6(uint32_t (&w)[6], int i, uint32_t code) {
  const int bit = 6 * i;
  w[bit / 32] |= code << (bit % 32);
  if (bit % 32 > 26) w[bit / 32 + 1] |= code >> (32 - bit % 32);
}

// E3M2 codes (low 6 bits of each byte) -> E4M3 codes of the same values (exact:
// every E3M2 value is an E4M3 value), four per dword.
__device__ __forceinline__ uint32_t e3m2x4_to_e4m3x4(uint32_t w) {
  uint32_t x = w & 0x1f1f1f1fu;
  uint32_t s = (w & 0x20202020u) << 2;
  uint32_t nrm = (x + 0x10101010u) << 1;
  uint32_t sub = __builtin_amdgcn_perm(0u, 0x24201800u, x);   // 0, 2^-4, 2^-3, 1.5*2^-3
  uint32_t m = ((x & 0x1c1c1c1cu) + 0x7c7c7c7cu) & 0x80808080u;
  uint32_t mask = m | (m - (m >> 7));
  return ((nrm & mask) | (sub & ~mask)) | s;
}

// ---------------------------------------------------------------------------
// R1 requant of the attention P tiles without rescaling P first.  With sh = 127 - sc,
// R1 encodes y = P * 2^sh: zero below F4M3 (the smallest float whose floorf(log2f())
// is >= -6), 448 from 448 up, RNE on the E4M3 grid in between.  The flush bound is moved
// to the P side (an exact power-of-two scaling): zero below F4M3 * 2^-sh -- for sh >= 120
// that bound is below 2^-126 and no nonzero P of an exponential (which returns 0 below
// 2^-126) reaches it.  The conversion then divides by its scale operand; it uses only that
// operand's exponent field (measured on gfx950: 1.5 acts as 1, 3.0 as 2, and a float with
// exponent field 0 as 2^-127), so (sc << 23) | 0x400000 is 2^(sc - 127) for every code,
// sc = 0 included.  The 448 saturation is applied to the packed codes: the conversion has
// no saturating form and returns 0x7f for a scaled value above 464 (values in (448, 464]
// round to 448); a P never exceeds its tile amax by more than a rounding residue and the
// amax scales into [256, 512), so every code is at most 0x7f and 0x7f -> 0x7e is exactly
// R1's saturation (three instructions per four codes instead of a min per value).
// ---------------------------------------------------------------------------
constexpr uint32_t kE4M3FlushBits = (120u << 23) | 0x7ffffeu;   // F4M3

struct PTileBounds {
  float flush, scale;
};

// flush = F4M3 * 2^(sc - 127) for sc >= 8, as the bit pattern (sc << 23) + (F4M3 bits -
// (127 << 23)) in wrapping 32-bit arithmetic.  For sc < 8 the same expression gives a
// negative float, a NaN pattern or (sc = 7) a subnormal below 2^-126, and no P >= 0 is
// below it except 0 itself (an exponential returns no subnormals): no flush, as R1 wants.
__device__ __forceinline__ PTileBounds p_tile_bounds(uint32_t sc) {
  PTileBounds b;
  b.flush = __uint_as_float((sc << 23) + (kE4M3FlushBits - (127u << 23)));
  b.scale = __uint_as_float((sc << 23) | 0x400000u);
  return b;
}

typedef short v2s_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float p_flush(float p, const PTileBounds& b) { return p < b.flush ? 0.0f : p; }

// Four already bounded values of one tile -> their E4M3 codes (byte i = value i).
__device__ __forceinline__ uint32_t cvt_pack4(float y0, float y1, float y2, float y3, float scale) {
  v2s_t pk;
  pk = __builtin_nondeterministic_value(pk);        // both halves are written below
  pk = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(pk, y0, y1, scale, false);
  pk = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(pk, y2, y3, scale, true);
  return __builtin_bit_cast(uint32_t, pk);
}

// The same, with the first conversion writing into y0's register (no longer needed once
// converted), which spares the register clear the form above gets (R1 P tiles; with the
// R2 tiles it measured slower).
__device__ __forceinline__ uint32_t cvt_pack4_in_place(float y0, float y1, float y2, float y3, float scale) {
  v2s_t pk = __builtin_bit_cast(v2s_t, y0);
  pk = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(pk, y0, y1, scale, false);
  pk = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(pk, y2, y3, scale, true);
  return __builtin_bit_cast(uint32_t, pk);
}

// Four P values (>= 0, finite, at most the tile amax) of one tile -> their R1 E4M3 codes
// (byte i = value i).
__device__ __forceinline__ uint32_t p_pack4(float p0, float p1, float p2, float p3, const PTileBounds& b) {
  const uint32_t w = cvt_pack4_in_place(p_flush(p0, b), p_flush(p1, b), p_flush(p2, b), p_flush(p3, b), b.scale);
  const uint32_t top = (w + 0x01010101u) >> 7;     // bit 0 of each byte: that byte was 0x7f
  return w ^ (top & 0x01010101u);                  // 0x7f -> 0x7e, other bytes unchanged
}

// R1 E4M3 codes of four already scaled values of any sign (byte i = value i), on the
// hardware conversion.  R1 (lib/golden/mx_fp_math.h:205-225, restated as
// orc_e4m3_encode in the oracle): E = floorf(log2f(|y|)); code 0 for |y| = 0, NaN, inf or
// E < -6; 0x7e with y's sign for E > 8; otherwise the mantissa rounded to nearest even at
// 3 bits (a carry raises E) and 0x7e for 480.  The same codes for every float:
// - |y| below F4M3 (floorf(log2f) < -6), zeros of either sign, NaN and infinities: R1
//   gives code 0; they are replaced by +0 before the conversion.
// - Where floorf(log2f(|y|)) is one above the exponent of |y| (a mantissa within a few
//   dozen ulps of the next power of two), R1 codes that power of two; round-to-nearest-
//   even to 3 mantissa bits rounds such a mantissa (above 1.9375) up to it as well.
// - F4M3 <= |y| < 2^-6 rounds to 2^-6 on the conversion's subnormal grid, R1's code 0x08.
// - R1 saturates at 448 (0x7e, sign kept); the conversion rounds |y| in (448, 464] to 448
//   and returns 0x7f / 0xff above, which is moved to 0x7e / 0xfe on the packed codes.
__device__ __forceinline__ float r1_keep(float y) {
  const float a = __builtin_fabsf(y);
  return (a >= __uint_as_float(kE4M3FlushBits) && a < __builtin_inff()) ? y : 0.0f;
}

__device__ __forceinline__ uint32_t e4m3_code4(float y0, float y1, float y2, float y3) {
  const uint32_t w = cvt_pack4(r1_keep(y0), r1_keep(y1), r1_keep(y2), r1_keep(y3), 1.0f);
  const uint32_t top = ((w & 0x7f7f7f7fu) + 0x01010101u) & 0x80808080u;   // that byte's low 7 bits were all 1
  return w ^ (top >> 7);
}

// ---------------------------------------------------------------------------
// Rule R2, the reference device kernels' P requant ("target-0", truncating;
// kernels/flash_attention_mx_gqa/flash_mx_impl.hpp:53-77, 366-388, 485-501), on P
// rounded to bf16 (the reference's P is bf16).  Scale code sc = the bf16 exponent field
// of the tile amax, clamped to <= 127 (se = sc - 127 <= 0).  Element: the bf16 P with
// its mantissa cut to 3 bits, flushed when its exponent is below se - 6 (or its field
// is 0).  P <= amax up to a rounding residue, so P / 2^se < 4 and the rule's saturation
// never applies; the cut value divided by 2^se is then an E4M3 normal, which the
// conversion encodes exactly.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t bf16_rne_bits(float x) {     // finite x >= 0: bf16 RNE, in the high half
  const uint32_t b = __float_as_uint(x);
  return (b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u;
}

__device__ __forceinline__ uint32_t r2_scale_code(float amax) {
  const uint32_t f = bf16_rne_bits(amax) >> 23;
  return f < 127u ? f : 127u;
}

struct PTileR2 {
  float flush, scale;
};

__device__ __forceinline__ PTileR2 p_tile_r2(uint32_t sc) {
  PTileR2 b;
  b.flush = __uint_as_float(sc >= 6u ? (sc - 6u) << 23 : 0u);   // 2^(se - 6)
  b.scale = __uint_as_float((sc << 23) | 0x400000u);             // 2^se (exponent field only)
  return b;
}

// bf16 P (as float bits) -> the value R2 encodes, before the division by 2^se.
__device__ __forceinline__ float r2_cut(uint32_t pb, const PTileR2& b) {
  const float t = __uint_as_float(pb & 0xfff00000u);
  return t < b.flush ? 0.0f : t;
}

}  // namespace mxfa
