"""CPU tests pinning the oracle's MX GEMM (exact accumulation of the reference MX GEMM's
tile semantics, C = sum_g 2^(SA[g][m] + SB[g][n] - 254) sum_{k in g} A[m][k] B[k][n]).

Pins: the reference's own MX GEMM golden (lib/golden/mx_golden.cpp, built into
oracle/_ref) on the operand range the reference's generator uses (codes below 2,
kernels/gemm_mxgemmini/gen_mxgemm_data.py:66-80 via lib/golden/golden.py:174-181), within
the golden's hardware truncation; exact power-of-two scale and group-additivity
properties that a wrong scale index or operand orientation breaks."""
import os
import subprocess

import numpy as np
import pytest

import oracle as O
from mxdata import rel_l2


def _codes(rng, shape, small=False):
    c = rng.integers(0, 256, shape).astype(np.uint8)
    if small:                                             # exponent field <= 7: |value| < 2
        c = (c & 0x87) | ((rng.integers(0, 8, shape).astype(np.uint8)) << 3)
    c[(c & 0x7F) == 0x7F] = 0x7E                          # no NaN codes
    return c


def _mx_golden(tmp, a, b, sa, sb):
    exe = O.ref_mx_golden_path()
    M, K = a.shape
    N = b.shape[1]
    names = []
    for i, x in enumerate((a, b, sa, sb)):
        path = os.path.join(tmp, f"g{i}.bin")
        np.ascontiguousarray(x, np.uint8).tofile(path)
        names.append(path)
    out = os.path.join(tmp, "c.bin")
    subprocess.run([exe, str(M), str(N), str(K), *names, out], check=True,
                   env={k: v for k, v in os.environ.items() if k != "MX_OUT_FMT"})
    return ((np.fromfile(out, np.uint16).astype(np.uint32) << 16).view(np.float32)).reshape(M, N).astype(np.float64)


@pytest.mark.skipif(O.ref_mx_golden_path() is None, reason="reference mx_golden not built here")
@pytest.mark.parametrize("M,N,K", [(64, 64, 64), (128, 64, 256)])
def test_gemm_oracle_vs_reference_mx_golden(M, N, K, tmp_path):
    rng = np.random.default_rng(M + N + K)
    a, b = _codes(rng, (M, K), small=True), _codes(rng, (K, N), small=True)
    sa = rng.integers(0x7B, 0x83, (K // 32, M)).astype(np.uint8)   # the reference generator's range
    sb = rng.integers(0x7B, 0x83, (K // 32, N)).astype(np.uint8)
    want = O.mx_gemm(a, sa, b, sb)
    got = _mx_golden(str(tmp_path), a, b, sa, sb)
    assert rel_l2(got, want) < 0.1, rel_l2(got, want)             # the golden truncates products to 3 bits
    # the planted mistake: B transposed (same shape when square) is far off
    if M == N:
        bad = O.mx_gemm(a, sa, np.ascontiguousarray(b.T), sb)
        assert rel_l2(got, bad) > 0.5


def test_gemm_oracle_scale_and_group_properties():
    rng = np.random.default_rng(3)
    M, N, K = 48, 40, 128
    a, b = _codes(rng, (M, K)), _codes(rng, (K, N))
    sa = rng.integers(110, 140, (K // 32, M)).astype(np.uint8)
    sb = rng.integers(110, 140, (K // 32, N)).astype(np.uint8)
    c = O.mx_gemm(a, sa, b, sb)
    # group additivity: the K range split into its 32-groups sums back exactly
    parts = [O.mx_gemm(a[:, 32 * g:32 * g + 32], sa[g:g + 1], b[32 * g:32 * g + 32], sb[g:g + 1]) for g in range(K // 32)]
    np.testing.assert_array_equal(c, sum(parts))
    # one scale code + 1 doubles exactly that (group, row) contribution and nothing else
    sa2 = sa.copy()
    sa2[2, 5] += 1
    d = O.mx_gemm(a, sa2, b, sb) - c
    np.testing.assert_array_equal(np.delete(d, 5, axis=0), 0.0)
    tol = 1e-13 * np.abs(c).max()                             # fp64 rounding of (C + part) - C
    np.testing.assert_allclose(d[5], parts[2][5], rtol=1e-12, atol=tol)
    sb2 = sb.copy()
    sb2[1, 7] -= 1
    d = O.mx_gemm(a, sa, b, sb2) - c
    np.testing.assert_array_equal(np.delete(d, 7, axis=1), 0.0)
    np.testing.assert_allclose(d[:, 7], -parts[1][:, 7] / 2, rtol=1e-12, atol=tol)
    # zero operand codes give exact zeros; E3M2 codes decode through the E3M2 table
    np.testing.assert_array_equal(O.mx_gemm(np.zeros_like(a), sa, b, sb), 0.0)
    a6 = (a & 0x3F).astype(np.uint8)
    c6 = O.mx_gemm(a6, sa, b, sb, a_fmt=O.FMT_E3M2)
    L = O.lib()
    t6 = np.array([L.orc_e3m2_decode(i & 0x3F) for i in range(256)])
    t8 = np.array([L.orc_e4m3_decode(i) for i in range(256)])
    A = t6[a6] * np.repeat(2.0 ** (sa.T.astype(np.float64) - 127), 32, axis=1)
    B = t8[b] * np.repeat(2.0 ** (sb.astype(np.float64) - 127), 32, axis=0)
    np.testing.assert_allclose(c6, A @ B, rtol=1e-12, atol=1e-300)
