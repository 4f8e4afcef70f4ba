"""ctypes binding of the CPU oracle (oracle/liboracle.so) and of the reference's
own lib/golden code built into oracle/_ref/ (when present).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker.  The product path
(radiance-kernels_amd/) never imports this module.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")

FMT_E4M3 = 0
FMT_E3M2 = 1
P_R1 = 0
P_R2 = 1


class AttnParams(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32), ("num_q_heads", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32),
        ("seq_q", ctypes.c_int32), ("seq_k", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("causal", ctypes.c_int32), ("q_pos0", ctypes.c_int32), ("window", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float), ("softcap", ctypes.c_float), ("v_fmt", ctypes.c_int32),
        ("p_rule", ctypes.c_int32),
    ]


def build():
    """Compile liboracle.so (and oracle/_ref when the reference tree exists)."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER
        u8p, f32p = P(ctypes.c_uint8), P(ctypes.c_float)
        L.orc_floor_log2f.argtypes = [ctypes.c_float]; L.orc_floor_log2f.restype = ctypes.c_int
        L.orc_log2_tables.argtypes = [P(ctypes.c_uint32), P(ctypes.c_uint32)]
        L.orc_f32_to_bf16.argtypes = [ctypes.c_float]; L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_e4m3_encode.argtypes = [ctypes.c_float]; L.orc_e4m3_encode.restype = ctypes.c_uint8
        L.orc_e4m3_decode.argtypes = [ctypes.c_uint8]; L.orc_e4m3_decode.restype = ctypes.c_float
        L.orc_e3m2_encode_bf16.argtypes = [ctypes.c_uint16]; L.orc_e3m2_encode_bf16.restype = ctypes.c_uint8
        L.orc_e3m2_decode.argtypes = [ctypes.c_uint8]; L.orc_e3m2_decode.restype = ctypes.c_float
        L.orc_e8m0_decode.argtypes = [ctypes.c_uint8]; L.orc_e8m0_decode.restype = ctypes.c_double
        L.orc_scale_code.argtypes = [ctypes.c_float, ctypes.c_int]; L.orc_scale_code.restype = ctypes.c_uint8
        L.orc_quantize_rows.argtypes = [f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, u8p, u8p]
        L.orc_quantize_cols.argtypes = [f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, u8p, u8p]
        L.orc_attention.argtypes = [P(AttnParams), u8p, u8p, u8p, u8p, u8p, u8p, f32p,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int, P(ctypes.c_int32), ctypes.c_int,
                                    ctypes.c_int]
        L.orc_attention.restype = ctypes.c_int
        L.orc_attention_trace.argtypes = [P(AttnParams), u8p, u8p, u8p, u8p, u8p, u8p, ctypes.c_int, ctypes.c_int64,
                                          ctypes.c_int64, ctypes.c_void_p, u8p, u8p, ctypes.c_void_p]
        L.orc_attention_trace.restype = ctypes.c_int
        L.orc_attention_dense.argtypes = [P(AttnParams), u8p, u8p, u8p, u8p, u8p, u8p, f32p,
                                          P(ctypes.c_int32), ctypes.c_int, ctypes.c_int]
        L.orc_attention_dense.restype = ctypes.c_int
        L.orc_check_log2_vs_libm.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
        L.orc_check_log2_vs_libm.restype = ctypes.c_int64
        L.orc_e4m3_encode_range.argtypes = [ctypes.c_uint32, ctypes.c_uint32, P(ctypes.c_uint8)]
        L.orc_e4m3_encode_array.argtypes = [f32p, ctypes.c_int64, u8p]
        L.orc_r4_encode.argtypes = [ctypes.c_float]; L.orc_r4_encode.restype = ctypes.c_uint8
        L.orc_r4_quantize_rows.argtypes = [f32p, ctypes.c_int64, ctypes.c_int64, u8p, u8p]
        L.orc_r4_check.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int]
        L.orc_r4_check.restype = ctypes.c_int64
        L.orc_r2_encode.argtypes = [ctypes.c_uint16, ctypes.c_int]; L.orc_r2_encode.restype = ctypes.c_uint8
        L.orc_r2_scale_exp.argtypes = [ctypes.c_float]; L.orc_r2_scale_exp.restype = ctypes.c_int
        L.orc_r2_encode_array.argtypes = [P(ctypes.c_uint16), P(ctypes.c_int32), ctypes.c_int64, u8p]
        L.orc_r2_quantize_rows.argtypes = [f32p, ctypes.c_int64, ctypes.c_int64, f32p, u8p, u8p]
        f64p = P(ctypes.c_double)
        L.orc_mx_gemm.argtypes = [u8p, u8p, u8p, u8p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                  ctypes.c_int, f64p, f64p]
        _lib = L
    return _lib


def _u8(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))


def _f32(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def log2_tables():
    thr = np.zeros(256, np.uint32)
    sub = np.zeros(23, np.uint32)
    lib().orc_log2_tables(thr.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                          sub.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)))
    return thr, sub


def floor_log2f(x):
    return lib().orc_floor_log2f(float(x))


def quantize_rows(x, fmt):
    """x: float32 [..., cols] -> (codes uint8 same shape, scales uint8 [..., cols/32])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    cols = x.shape[-1]
    rows = x.size // cols
    codes = np.empty(x.shape, np.uint8)
    scales = np.empty(x.shape[:-1] + (cols // 32,), np.uint8)
    lib().orc_quantize_rows(_f32(x), rows, cols, fmt, _u8(codes), _u8(scales))
    return codes, scales


def quantize_cols(x, fmt):
    """x: float32 [..., rows, cols], blocks of 32 along rows per matrix ->
    (codes same shape, scales [..., rows/32, cols])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape[-2], x.shape[-1]
    mats = x.size // (rows * cols)
    codes = np.empty(x.shape, np.uint8)
    scales = np.empty(x.shape[:-2] + (rows // 32, cols), np.uint8)
    xf = x.reshape(mats, rows, cols)
    cf = codes.reshape(mats, rows, cols)
    sf = scales.reshape(mats, rows // 32, cols)
    for m in range(mats):
        lib().orc_quantize_cols(_f32(xf[m]), rows, cols, fmt, _u8(cf[m]), _u8(sf[m]))
    return codes, scales


def r4_quantize_rows(x):
    """Rule R4 (the reference's SIMT block quantizer) over 32-blocks along the last axis."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    cols = x.shape[-1]
    rows = x.size // cols
    codes = np.empty(x.shape, np.uint8)
    scales = np.empty(tuple(x.shape[:-1]) + (cols // 32,), np.uint8)
    lib().orc_r4_quantize_rows(_f32(x), rows, cols, _u8(codes), _u8(scales))
    return codes, scales


def e4m3_encode(x):
    """R1 E4M3 codes of already scaled float32 values (same shape as x)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().orc_e4m3_encode_array(_f32(x), x.size, _u8(out))
    return out


def r2_encode(bf16, se):
    """Rule R2 element codes of bf16 bit patterns (uint16) with block exponents se (int),
    broadcast against each other."""
    b, s = np.broadcast_arrays(np.asarray(bf16, np.uint16), np.asarray(se, np.int32))
    b, s = np.ascontiguousarray(b), np.ascontiguousarray(s)
    out = np.empty(b.shape, np.uint8)
    lib().orc_r2_encode_array(b.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
                              s.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), b.size, _u8(out))
    return out


def r2_quantize_rows(p):
    """Rule R2 over 32-blocks along the last axis of fp32 P: returns (P rounded to bf16 as
    float32, codes, scale codes)."""
    p = np.ascontiguousarray(p, dtype=np.float32)
    cols = p.shape[-1]
    rows = p.size // cols
    pb = np.empty(p.shape, np.float32)
    codes = np.empty(p.shape, np.uint8)
    scales = np.empty(tuple(p.shape[:-1]) + (cols // 32,), np.uint8)
    lib().orc_r2_quantize_rows(_f32(p), rows, cols, _f32(pb), _u8(codes), _u8(scales))
    return pb, codes, scales


def mx_gemm(a, sa, b, sb, a_fmt=FMT_E4M3, b_fmt=FMT_E4M3, with_abs=False):
    """Exact MX GEMM (float64): a [M][K], sa [K/32][M], b [K][N], sb [K/32][N] codes ->
    C [M][N] (and sum |term| per element when with_abs)."""
    a, sa, b, sb = (np.ascontiguousarray(x, dtype=np.uint8) for x in (a, sa, b, sb))
    M, K = a.shape
    N = b.shape[1]
    assert b.shape[0] == K and K % 32 == 0 and sa.shape == (K // 32, M) and sb.shape == (K // 32, N)
    c = np.empty((M, N), np.float64)
    ab = np.empty((M, N), np.float64) if with_abs else None
    f64p = ctypes.POINTER(ctypes.c_double)
    lib().orc_mx_gemm(_u8(a), _u8(sa), _u8(b), _u8(sb), M, N, K, a_fmt, b_fmt, c.ctypes.data_as(f64p),
                      ab.ctypes.data_as(f64p) if with_abs else None)
    return (c, ab) if with_abs else c


def make_params(B, Hq, Hkv, Sq, Sk, D, causal=False, q_pos0=0, window=0, scale=None, softcap=0.0, v_fmt=FMT_E4M3,
                p_rule=P_R1):
    return AttnParams(B, Hq, Hkv, Sq, Sk, D, int(causal), q_pos0, window,
                      float(scale if scale is not None else 1.0 / np.sqrt(D)), float(softcap), v_fmt, p_rule)


def attention(p, q, qs, k, ks, v, vs, block_n, split_len=0, heads=None, nthreads=None, out=None, n_parts=0):
    """Streaming MX attention oracle.  Returns fp32 O [B][Hq][Sq][D] (heads not listed are 0).
    n_parts > 0: that many interleaved partials (partial i = key blocks i, i + n_parts, ...);
    split_len > 0: contiguous chunks of split_len keys; partials merged by log-sum-exp."""
    if nthreads is None:
        nthreads = os.cpu_count() or 1
    arrs = [np.ascontiguousarray(a, dtype=np.uint8) for a in (q, qs, k, ks, v, vs)]
    o = out if out is not None else np.zeros((p.batch, p.num_q_heads, p.seq_q, p.head_dim), np.float32)
    hp, nh = None, 0
    if heads is not None:
        h = np.ascontiguousarray(np.asarray(heads, dtype=np.int32))
        hp, nh = h.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), len(h)
    rc = lib().orc_attention(ctypes.byref(p), *[_u8(a) for a in arrs], _f32(o), block_n, split_len, n_parts, hp, nh,
                                 nthreads)
    if rc != 0:
        raise ValueError("orc_attention rejected its arguments")
    return o


def attention_trace(p, q, qs, k, ks, v, vs, block_n, bh, qi):
    """Stages of one query row's streaming pass (orc_attention_trace): dict with S [Sk] (natural
    units, double, -inf masked), codes [Sk], scales [Sk/32], m and l [n_blocks] after each block."""
    arrs = [np.ascontiguousarray(a, dtype=np.uint8) for a in (q, qs, k, ks, v, vs)]
    Sk = p.seq_k
    nblk = (Sk + block_n - 1) // block_n
    S = np.full(Sk, np.nan, np.float64)
    codes = np.zeros(Sk, np.uint8)
    scales = np.zeros(Sk // 32, np.uint8)
    ml = np.zeros((nblk, 2), np.float64)
    rc = lib().orc_attention_trace(ctypes.byref(p), *[_u8(a) for a in arrs], block_n, bh, qi, S.ctypes.data_as(ctypes.c_void_p), _u8(codes),
                                   _u8(scales), ml.ctypes.data_as(ctypes.c_void_p))
    if rc != 0:
        raise ValueError("orc_attention_trace rejected its arguments")
    return {"S": S, "codes": codes, "scales": scales, "m": ml[:, 0], "l": ml[:, 1]}


def attention_dense(p, q, qs, k, ks, v, vs, heads=None, nthreads=None):
    if nthreads is None:
        nthreads = os.cpu_count() or 1
    arrs = [np.ascontiguousarray(a, dtype=np.uint8) for a in (q, qs, k, ks, v, vs)]
    o = np.zeros((p.batch, p.num_q_heads, p.seq_q, p.head_dim), np.float32)
    hp, nh = None, 0
    if heads is not None:
        h = np.ascontiguousarray(np.asarray(heads, dtype=np.int32))
        hp, nh = h.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), len(h)
    rc = lib().orc_attention_dense(ctypes.byref(p), *[_u8(a) for a in arrs], _f32(o), hp, nh, nthreads)
    if rc != 0:
        raise ValueError("orc_attention_dense rejected its arguments")
    return o


# ------------------------------------------------------------------ reference
_ref = None


def ref_available():
    return os.path.exists(os.path.join(REF_DIR, "libmxref.so"))


def ref():
    """The reference's lib/golden element rules compiled from its own sources."""
    global _ref
    if _ref is None:
        R = ctypes.CDLL(os.path.join(REF_DIR, "libmxref.so"))
        P = ctypes.POINTER
        R.ref_e4m3_encode_range.argtypes = [ctypes.c_uint32, ctypes.c_uint32, P(ctypes.c_uint8)]
        R.ref_e4m3_encode_array.argtypes = [P(ctypes.c_float), ctypes.c_int64, P(ctypes.c_uint8)]
        R.ref_e4m3_decode.argtypes = [ctypes.c_uint8]; R.ref_e4m3_decode.restype = ctypes.c_float
        R.ref_e3m2_decode.argtypes = [ctypes.c_uint8]; R.ref_e3m2_decode.restype = ctypes.c_float
        R.ref_e8m0_decode.argtypes = [ctypes.c_uint8]; R.ref_e8m0_decode.restype = ctypes.c_float
        R.ref_e3m2_encode_bf16.argtypes = [ctypes.c_uint16]; R.ref_e3m2_encode_bf16.restype = ctypes.c_uint8
        R.ref_f32_to_bf16_array.argtypes = [P(ctypes.c_float), ctypes.c_int64, P(ctypes.c_uint16)]
        _ref = R
    return _ref


def ref_mx_golden_path():
    p = os.path.join(REF_DIR, "mx_golden")
    return p if os.path.exists(p) else None
