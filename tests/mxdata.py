"""Shared test helpers: synthetic MX operands quantized by the oracle."""
import numpy as np

import oracle as O


def quantize_qkv(Q, K, V, v_fmt=O.FMT_E4M3):
    """Q [B,Hq,Sq,D], K/V [B,Hkv,Sk,D] fp32 -> codes/scales in the C-ABI layouts
    (Q, K blocked along D; V blocked along the key axis)."""
    q, qs = O.quantize_rows(Q, O.FMT_E4M3)
    k, ks = O.quantize_rows(K, O.FMT_E4M3)
    v, vs = O.quantize_cols(V, v_fmt)
    return q, qs, k, ks, v, vs


def normal_inputs(B, Hq, Hkv, Sq, Sk, D, seed=0, outlier_p=0.0, outlier_mul=20.0, q_mul=1.0):
    rng = np.random.default_rng(seed)
    Q = rng.standard_normal((B, Hq, Sq, D), dtype=np.float32) * np.float32(q_mul)
    K = rng.standard_normal((B, Hkv, Sk, D), dtype=np.float32)
    V = rng.standard_normal((B, Hkv, Sk, D), dtype=np.float32)
    if outlier_p > 0:
        for X in (Q, K, V):
            X[rng.random(X.shape) < outlier_p] *= np.float32(outlier_mul)
    return Q, K, V


def dequant_rows(codes, scales, fmt):
    L = O.lib()
    if fmt == O.FMT_E4M3:
        tab = np.array([L.orc_e4m3_decode(c) for c in range(256)], np.float64)
    else:
        tab = np.array([L.orc_e3m2_decode(c & 0x3F) for c in range(256)], np.float64)
    return tab[codes] * np.repeat(2.0 ** (scales.astype(np.float64) - 127), 32, axis=-1)


def dequant_cols(codes, scales, fmt):
    L = O.lib()
    if fmt == O.FMT_E4M3:
        tab = np.array([L.orc_e4m3_decode(c) for c in range(256)], np.float64)
    else:
        tab = np.array([L.orc_e3m2_decode(c & 0x3F) for c in range(256)], np.float64)
    return tab[codes] * np.repeat(2.0 ** (scales.astype(np.float64) - 127), 32, axis=-2)


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))
