"""CPU tests pinning the oracle's MX element and scale rules.

Pins, in order of strength:
  * committed fixtures written from the reference's own lib/golden code
    (tests/golden/make_golden.py): decode tables, the E3M2 encoder over all
    65536 bf16 patterns, the E4M3 encoder on edge cases, and the mx_golden
    CLI's block-32 requant post-pass (codes + E8M0 scales), and rule R4 from the
    reference's golden.py bit primitives (tests/golden/make_r4_golden.py);
  * the reference's compiled code itself (oracle/_ref) where it was built;
  * closed forms: the OCP E4M3/E3M2 grids, libm's floorf(log2f(x)) over every
    positive float, and scale-range invariants.
"""
import ctypes
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_decode_tables_match_reference_fixture():
    z = np.load(os.path.join(GOLD, "decode_tables.npz"))
    L = O.lib()
    e4 = np.array([L.orc_e4m3_decode(c) for c in range(256)], np.float32)
    e3 = np.array([L.orc_e3m2_decode(c) for c in range(64)], np.float32)
    e8 = np.array([L.orc_e8m0_decode(c) for c in range(255)], np.float64)
    np.testing.assert_array_equal(e4, z["e4m3"])
    np.testing.assert_array_equal(e3, z["e3m2"])
    np.testing.assert_array_equal(e8.astype(np.float32), z["e8m0"])
    assert np.isnan(L.orc_e8m0_decode(255))


def test_decode_closed_forms():
    """OCP E4M3: bias 7, subnormal step 2^-9, max 448; E3M2: bias 3, step 2^-4, max 28."""
    L = O.lib()
    assert L.orc_e4m3_decode(0x7E) == 448.0 and L.orc_e4m3_decode(0x08) == 2.0 ** -6
    assert L.orc_e4m3_decode(0x01) == 2.0 ** -9 and L.orc_e4m3_decode(0x38) == 1.0
    assert L.orc_e3m2_decode(0x1F) == 28.0 and L.orc_e3m2_decode(0x01) == 0.0625
    assert L.orc_e3m2_decode(0x0C) == 1.0 and L.orc_e3m2_decode(0x3F) == -28.0


def test_e3m2_encoder_all_bf16_vs_fixture():
    want = np.fromfile(os.path.join(GOLD, "e3m2_encode.bin"), np.uint8)
    L = O.lib()
    got = np.array([L.orc_e3m2_encode_bf16(b) for b in range(65536)], np.uint8)
    np.testing.assert_array_equal(got, want)


def test_e3m2_encoder_is_nearest_on_grid():
    """Independent check: in the scaled range the E3M2 code is the nearest E3M2 value
    of the bf16 input (ties to even mantissa), up to the pipeline's E4M2 double rounding."""
    L = O.lib()
    grid = np.array([L.orc_e3m2_decode(c) for c in range(32)], np.float64)
    rng = np.random.default_rng(1)
    for v in rng.uniform(0.3, 27.0, 2000).astype(np.float32):
        b = L.orc_f32_to_bf16(float(v))
        x = float(np.uint32(b << 16).view(np.float32))
        code = L.orc_e3m2_encode_bf16(b)
        err = abs(grid[code] - x)
        assert err <= np.min(np.abs(grid - x)) + 1e-12 or abs(err - np.min(np.abs(grid - x))) < x * 2 ** -3


def test_e4m3_encoder_edge_fixture():
    z = np.load(os.path.join(GOLD, "e4m3_encode.npz"))
    L = O.lib()
    x = z["x"]
    got = np.array([L.orc_e4m3_encode(float(v)) for v in x], np.uint8)
    bad = np.nonzero(got != z["code"])[0]
    assert len(bad) == 0, [(float(x[i]), hex(got[i]), hex(z["code"][i])) for i in bad[:10]]


def test_e4m3_encoder_closed_form_on_grid():
    """Every finite E4M3 value in [2^-6, 448] encodes to its own code (exact grid points)."""
    L = O.lib()
    for c in range(256):
        e = (c >> 3) & 15
        if e == 0 or (c & 0x7F) == 0x7F:
            continue
        assert L.orc_e4m3_encode(L.orc_e4m3_decode(c)) == c


def test_floor_log2f_exhaustive_vs_libm():
    """Every positive finite float: table-based floor(log2) == libm floorf(log2f(x))."""
    L = O.lib()
    N, nt = 0x7F800000, 32
    step = N // nt + 1
    with ThreadPoolExecutor(min(8, os.cpu_count() or 1)) as ex:
        bad = sum(ex.map(lambda i: L.orc_check_log2_vs_libm(1 + i * step, min(N, 1 + (i + 1) * step)), range(nt)))
    assert bad == 0


def test_log2_table_shape():
    """Thresholds sit just below powers of two and are monotone in |e|."""
    thr, sub = O.log2_tables()
    for E in range(1, 255):
        assert thr[E] == 0x800000 or thr[E] >= 0x7FFF00
    assert thr[127] == 0x800000 and thr[126] == 0x800000    # e = 0, -1: log2 near 1 and 0 is exact enough
    assert thr[127 + 4] == 0x7FFFFE and thr[127 + 64] == 0x7FFFD4


@pytest.mark.skipif(not O.ref_available(), reason="reference lib/golden not built here")
def test_e4m3_encoder_vs_reference_whole_range():
    """Every float in [2^-10, 2^10) of both signs vs the reference's compiled fp8_e4m3_to_code."""
    L, R = O.lib(), O.ref()
    lo, hi = int(np.float32(2.0 ** -10).view(np.uint32)), int(np.float32(2.0 ** 10).view(np.uint32))
    for sign in (0, 0x80000000):
        for b0 in range(lo, hi, 1 << 24):
            cnt = min(1 << 24, hi - b0)
            a = np.empty(cnt, np.uint8)
            r = np.empty(cnt, np.uint8)
            L.orc_e4m3_encode_range(b0 | sign, cnt, a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)))
            R.ref_e4m3_encode_range(b0 | sign, cnt, r.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)))
            assert int((a != r).sum()) == 0


@pytest.mark.skipif(not O.ref_available(), reason="reference lib/golden not built here")
def test_bf16_rounding_vs_reference():
    L, R = O.lib(), O.ref()
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * np.float32(1e3),
                        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-45, 3.4e38], np.float32)])
    x = np.ascontiguousarray(x)
    r = np.empty(len(x), np.uint16)
    R.ref_f32_to_bf16_array(x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), len(x),
                            r.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)))
    got = np.array([L.orc_f32_to_bf16(float(v)) for v in x], np.uint16)
    np.testing.assert_array_equal(got, r)


def test_requant_postpass_vs_mx_golden_fixture():
    """The reference CLI's MX_OUT_FMT=0 post-pass (mx_golden.cpp:146-190) on its own bf16 C."""
    z = np.load(os.path.join(GOLD, "requant_postpass.npz"))
    n = len([k for k in z.files if k.startswith("C")])
    assert n >= 3
    for i in range(n):
        C = (z[f"C{i}"].astype(np.uint32) << 16).view(np.float32)
        codes, scales = O.quantize_rows(C, O.FMT_E4M3)
        np.testing.assert_array_equal(scales, z[f"scales{i}"])
        np.testing.assert_array_equal(codes, z[f"codes{i}"])


def test_scale_code_invariants():
    """amax == 0 -> 0; otherwise amax / 2^(code-127) in [256, 512) (E4M3) / [16, 32) (E3M2)
    except in the one-ulp log2f window just below a power of two, and clamped to [0, 254]."""
    L = O.lib()
    rng = np.random.default_rng(7)
    assert L.orc_scale_code(0.0, 0) == 0 and L.orc_scale_code(0.0, 1) == 0
    for a in (rng.standard_normal(5000).astype(np.float32) ** 2 * np.float32(2.0) ** rng.integers(-100, 100, 5000)):
        if not np.isfinite(a) or a == 0:
            continue
        for fmt, lo in ((0, 256.0), (1, 16.0)):
            c = L.orc_scale_code(float(a), fmt)
            r = float(a) / 2.0 ** (c - 127)
            if 0 < c < 254:
                assert lo * (1 - 2 ** -20) <= r < 2 * lo
    assert L.orc_scale_code(1e-42, 0) == 0 and L.orc_scale_code(3.0e38, 0) == 127 - 8 + 127


def test_quantize_rows_cols_roundtrip_error_bound():
    """Dequantized MX values are within half an E4M3 ulp (relative 2^-4) of the input for
    elements within 2^-6 of the block scale range, and blocks are independent."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal((64, 128)).astype(np.float32)
    codes, scales = O.quantize_rows(x, O.FMT_E4M3)
    L = O.lib()
    scale = np.repeat(2.0 ** (scales.astype(np.float64) - 127), 32, axis=1)
    dec = np.vectorize(lambda c: L.orc_e4m3_decode(int(c)))(codes) * scale
    y = np.abs(x) / scale
    normal = (y >= 2.0 ** -6) & (y <= 448.0)
    assert np.all(np.abs(dec - x)[normal] <= np.abs(x)[normal] * 2.0 ** -4 + 1e-30)
    sat = y > 464.0
    assert np.all(np.abs(dec[sat]) == 448.0 * scale[sat])
    assert np.all(dec[y < 2.0 ** -7] == 0.0)
    # column blocking equals row blocking of the transpose
    c2, s2 = O.quantize_cols(np.ascontiguousarray(x.T), O.FMT_E4M3)
    np.testing.assert_array_equal(c2, codes.T)
    np.testing.assert_array_equal(s2, scales.T)


def _bits(x):
    return int(np.array(x, np.float32).view(np.uint32))


def test_r4_element_rule_equals_r1_from_2_pow_minus_6():
    """Rule R4 (simt_quant) rounds and saturates like R1 wherever R1 does not flush: every
    float in [2^-6, 2^10) of either sign gets the same E4M3 code, and a strided sample of
    the saturating range above."""
    L = O.lib()
    lo, hi = _bits(2.0 ** -6), _bits(2.0 ** 10)                   # exhaustive up to 1024
    assert L.orc_r4_check(lo, hi, 0) == 0
    assert L.orc_r4_check(lo | 0x80000000, hi | 0x80000000, 0) == 0
    for b in range(hi, 0x7F800000, 9973):                         # saturation region, sampled
        assert L.orc_r4_check(b, b + 1, 0) == 0 and L.orc_r4_check(b | 0x80000000, (b | 0x80000000) + 1, 0) == 0


def test_r4_element_rule_keeps_subnormals_on_the_2_pow_minus_9_grid():
    """Below 2^-6 R4 keeps E4M3 subnormals: the code is round-half-even of |y| * 512
    (checked over every float in [2^-24, 2^-6), both signs, and the smallest values)."""
    L = O.lib()
    lo, hi = _bits(2.0 ** -24), _bits(2.0 ** -6)
    assert L.orc_r4_check(lo, hi, 1) == 0
    assert L.orc_r4_check(lo | 0x80000000, hi | 0x80000000, 1) == 0
    assert L.orc_r4_check(0, 4096, 1) == 0
    assert L.orc_r4_encode(2.0 ** -10) == 0                    # tie -> even (0)
    assert L.orc_r4_encode(3 * 2.0 ** -10) == 2                # tie -> even (2)
    assert L.orc_r4_encode(7.75 * 2.0 ** -9) == 0x08           # rounds up to 2^-6, a normal code


def test_r4_scale_is_ceil_log2_amax_over_448():
    """R4's block scale: the smallest e with amax <= 448 * 2^e (exact in double), code
    e + 127 clamped to [0, 254]; amax = 0 gives code 0.  Includes amax exactly at and just
    around 448 * 2^k."""
    rng = np.random.default_rng(500)
    amaxes = list(np.exp2(rng.uniform(-118, 127, 4000)).astype(np.float32))
    for k in range(-120, 120, 7):
        t = np.float32(448.0 * 2.0 ** k)
        amaxes += [t, np.nextafter(t, np.float32(0)), np.nextafter(t, np.float32(np.inf))]
    amaxes = [a for a in amaxes if np.isfinite(a) and a >= np.float32(2.0 ** -126)]
    x = np.zeros((len(amaxes), 32), np.float32)
    x[:, 7] = -np.array(amaxes, np.float32)
    x[:, 3] = np.array(amaxes, np.float32) * np.float32(0.25)
    _, sc = O.r4_quantize_rows(x)
    for a, s in zip(amaxes, sc[:, 0]):
        e = int(np.ceil(np.log2(float(a) / 448.0)))
        while 448.0 * 2.0 ** e < float(a):
            e += 1
        while 448.0 * 2.0 ** (e - 1) >= float(a):
            e -= 1
        assert s == min(max(e + 127, 0), 254), (a, s, e)
    _, sc0 = O.r4_quantize_rows(np.zeros((1, 32), np.float32))
    assert sc0[0, 0] == 0


def test_r4_matches_reference_golden_fixture():
    """R4 against the reference's own bit primitives (lib/golden/golden.py block_exp,
    pow2_neg_e, fp8_code_rshift, composed per block as kernels/simt_quant/gen_quant.py:54-70;
    tests/golden/make_r4_golden.py): blocks whose amax is an fp32 subnormal or a normal below
    2^-120 (where the reference's (127 - e) << 23 multiplier word wraps), the normal range
    and amax at / around 448 * 2^k -- codes and scales bit for bit."""
    z = np.load(os.path.join(GOLD, "r4_blocks.npz"))
    codes, scales = O.r4_quantize_rows(z["x"])
    np.testing.assert_array_equal(scales.reshape(-1), z["scales"])
    np.testing.assert_array_equal(codes, z["codes"])
    # the fixture reaches the wrapped multiplier: scale code 0 with nonzero inputs
    assert np.any((z["scales"] == 0) & np.any(z["x"] != 0, axis=1))


# ---- rule R2: the reference device kernels' truncating P requant
# (kernels/flash_attention_mx_gqa/flash_mx_impl.hpp:53-77)

def _all_bf16_finite():
    b = np.arange(0, 0x10000, dtype=np.uint32)
    b = b[((b >> 7) & 0xFF) != 0xFF]                      # finite patterns of both signs
    return b.astype(np.uint16), (b << 16).view(np.float32).astype(np.float64)


@pytest.mark.parametrize("se", [0, -1, -3, -6, -7, -40, -119, -120, -121, -126, -127])
def test_r2_element_rule_is_truncation_on_the_e4m3_grid(se):
    """Every finite bf16 with block exponent se: the code's value is |v| * 2^-se with its
    binary mantissa cut to 3 bits (floor), 0 below 2^-6 or for a zero exponent field,
    448 from 2^9 up or where the cut value is 480; the sign is kept."""
    b, v = _all_bf16_finite()
    codes = O.r2_encode(b, se)
    L = O.lib()
    dec = np.array([L.orc_e4m3_decode(int(c)) for c in range(256)], np.float64)[codes]
    y = np.abs(v) * 2.0 ** -se
    e = np.floor(np.log2(np.where(y > 0, y, 1.0)))
    t = np.floor(y / 2.0 ** e * 8.0) / 8.0 * 2.0 ** e       # 3-bit truncation
    want = np.where(y >= 2.0 ** -6, np.minimum(np.where(y >= 512.0, 448.0, t), 448.0), 0.0)
    want[((b >> 7) & 0xFF) == 0] = 0.0                      # bf16 zero / subnormal
    np.testing.assert_array_equal(np.abs(dec), want)
    nz = codes != 0
    np.testing.assert_array_equal((codes[nz] >> 7).astype(bool), v[nz] < 0)


def test_r2_element_rule_equals_the_reference_integer_derivation():
    """The reference's own second formulation (kernels/flash_attention_mx/flash_mx_impl.hpp:
    196-216, e4m3_pack4): for P >= 0 no larger than 2^(se+1), code = t if t >= 8 else 0 with
    t = bits[14:4] - ((120 + se) << 3), se clamped to >= -120 by its callers."""
    b = np.arange(0, 0x7F80, dtype=np.uint32)               # +0 .. largest finite positive
    for se in range(-120, 1):
        keep = ((b >> 7) & 0xFF) - 127 <= se                # E <= 0: value below 2^(se+1)
        bb = b[keep]
        t = ((bb >> 4) & 0x7FF).astype(np.int64) - ((120 + se) << 3)
        want = np.where(t >= 8, t, 0).astype(np.uint8)
        np.testing.assert_array_equal(O.r2_encode(bb.astype(np.uint16), se), want)


def test_r2_scale_maps_the_bf16_block_max_into_one_to_two():
    L = O.lib()
    rng = np.random.default_rng(21)
    a = (rng.random(20000) * 2.0 ** rng.integers(-126, 1, 20000)).astype(np.float32)
    a = a[(a >= np.float32(2.0 ** -126)) & (a <= 1)]      # normal: a subnormal max gives se = -127
    se = np.array([L.orc_r2_scale_exp(float(x)) for x in a])
    hb = np.array([L.orc_f32_to_bf16(float(x)) for x in a], np.uint32)
    mb = (hb << 16).view(np.float32).astype(np.float64)
    r = mb / 2.0 ** se
    assert np.all((r >= 1.0) & (r < 2.0))
    assert L.orc_r2_scale_exp(1.0) == 0 and L.orc_r2_scale_exp(0.5) == -1
    assert L.orc_r2_scale_exp(float(np.float32(1.0 - 2.0 ** -10))) == 0   # bf16 rounds up to 1
    assert L.orc_r2_scale_exp(float(np.float32(0.5 - 2.0 ** -12))) == -1
    assert L.orc_r2_scale_exp(7.5) == 0                                   # clamped to <= 0
    assert L.orc_r2_scale_exp(0.0) == -127                                # code 0


def test_r2_blocks_target_zero():
    """R2 over P blocks: P is rounded to bf16, each nonzero block's largest code decodes into
    [1, 2) (the 'target-0' exponent), codes never exceed it, and an all-zero block has scale
    and codes 0."""
    rng = np.random.default_rng(22)
    p = np.exp2(-rng.exponential(6.0, (512, 128))).astype(np.float32)
    p[3] = 0.0
    p[5, 32:64] = 0.0
    p[7, :32] *= np.float32(2.0 ** -100)
    pb, codes, scales = O.r2_quantize_rows(p)
    L = O.lib()
    hb = np.array([L.orc_f32_to_bf16(float(x)) for x in p.ravel()], np.uint32).reshape(p.shape)
    np.testing.assert_array_equal(pb, (hb << 16).view(np.float32))
    dec = np.array([L.orc_e4m3_decode(int(c)) for c in range(256)], np.float64)[codes]
    blk = dec.reshape(512, 4, 32).max(axis=2)
    nzb = pb.reshape(512, 4, 32).max(axis=2) > 0
    assert np.all((blk[nzb] >= 1.0) & (blk[nzb] < 2.0))
    assert np.all(scales[~nzb] == 0) and np.all(blk[~nzb] == 0)
    assert scales[3].tolist() == [0, 0, 0, 0] and scales[5, 1] == 0
    # dequantized P never exceeds the bf16 P and is within 2^-3 of it where not flushed
    deq = dec * np.repeat(2.0 ** (scales.astype(np.float64) - 127), 32, axis=1)
    assert np.all(deq <= pb)
    kept = codes != 0
    assert np.all(pb[kept] - deq[kept] < pb[kept] * 2.0 ** -3)
