"""GPU parity of the MX GEMM (mxfa_gemm) against the oracle's exact accumulation: every
element within 2^-8 of the sum of its absolute terms (the scaled MFMA sums groups of 8
products in a 14-bit window; fp32 accumulation), rel-L2 within 1e-3; E3M2 operands; real
data quantized on the GPU; the R1 requant of C bit-exact."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import mxfa  # noqa: E402
import oracle as O  # noqa: E402
from gpuhelp import DEV, np_, sweep_seeds  # noqa: E402
from mxdata import rel_l2  # noqa: E402

pytestmark = pytest.mark.gpu


def _codes(rng, shape, fmt):
    c = rng.integers(0, 256, shape).astype(np.uint8)
    if fmt == mxfa.FMT_E3M2:
        return (c & 0x3F).astype(np.uint8)
    c[(c & 0x7F) == 0x7F] = 0x7E
    return c


def run_gemm(M, N, K, seed, a_fmt=mxfa.FMT_E4M3, b_fmt=mxfa.FMT_E4M3, srange=(112, 142)):
    print(f"gemm M{M} N{N} K{K} fmt {a_fmt}/{b_fmt} seed {seed}", flush=True)
    rng = np.random.default_rng(seed)
    a, b = _codes(rng, (M, K), a_fmt), _codes(rng, (K, N), b_fmt)
    sa = rng.integers(*srange, (K // 32, M)).astype(np.uint8)
    sb = rng.integers(*srange, (K // 32, N)).astype(np.uint8)
    dev = [torch.from_numpy(x).to(DEV) for x in (a, sa, b, sb)]
    out = torch.full((M, N), float("nan"), dtype=torch.float32, device=DEV)
    mxfa.gemm(dev[0], dev[1], dev[2], dev[3], a_fmt, b_fmt, out=out)
    torch.cuda.synchronize()
    c = np_(out).astype(np.float64)
    want, ab = O.mx_gemm(a, sa, b, sb, a_fmt, b_fmt, with_abs=True)
    assert np.all(np.isfinite(c)), "coverage"
    err = np.abs(c - want)
    worst = float((err / np.maximum(ab, 1e-300)).max())
    print(f"   rel-L2 {rel_l2(c, want):.2e}, max err / sum|terms| {worst:.2e}", flush=True)
    assert np.all(err <= ab * 2.0 ** -8 + 1e-38)
    assert rel_l2(c, want) <= 1e-3
    return c


@pytest.mark.parametrize("M,N,K", [(64, 64, 64), (256, 256, 256), (128, 128, 5632), (48, 80, 192),
                                   (512, 384, 1024), (272, 528, 320)])
def test_gemm_matches_oracle(M, N, K):
    run_gemm(M, N, K, seed=M + 3 * N + 7 * K)


@pytest.mark.parametrize("i", sweep_seeds(range(12), "MXFA_GEMM_SEEDS"))
def test_gemm_sweep(i, monkeypatch):
    """Seeded shapes (M = 16 .. 1,024, N = 16 .. 1,104, K = 64 .. 2,496) with E4M3 or E3M2
    operands through each kernel path (the default choice -- skinny for M <= 128, else the
    LDS-DMA kernel for E4M3 with K % 128 == 0 -- MXFA_GEMM=big or =reg); MXFA_GEMM_SEEDS=0-300
    runs the exploratory length."""
    rng = np.random.default_rng(31000 + i)
    M = 16 * int(rng.choice([1, 2, 3, 4, 5, 7, 8, 9, 16, 17, 33, 64]))
    N = 16 * int(rng.integers(1, 70))
    K = 64 * int(rng.integers(1, 40))
    af = int(rng.choice([mxfa.FMT_E4M3, mxfa.FMT_E4M3, mxfa.FMT_E3M2]))
    bf = int(rng.choice([mxfa.FMT_E4M3, mxfa.FMT_E4M3, mxfa.FMT_E3M2]))
    mode = str(rng.choice(["", "big", "reg"]))
    if mode:
        monkeypatch.setenv("MXFA_GEMM", mode)
    else:
        monkeypatch.delenv("MXFA_GEMM", raising=False)
    run_gemm(M, N, K, seed=31000 + i, a_fmt=af, b_fmt=bf)


def test_gemm_e3m2_operands_and_wide_scales():
    run_gemm(256, 128, 512, seed=11, a_fmt=mxfa.FMT_E3M2)
    run_gemm(128, 256, 256, seed=12, b_fmt=mxfa.FMT_E3M2)
    run_gemm(144, 336, 384, seed=14, a_fmt=mxfa.FMT_E3M2, b_fmt=mxfa.FMT_E3M2)
    # scale sums 2^-94 .. 2^84: every product and sum stays in fp32's normal range
    run_gemm(128, 128, 256, seed=13, srange=(80, 170))


def test_gemm_real_data_and_requant():
    """X W with X, W quantized on the GPU (R1; X along K, W along K per column) is within
    the MX error of the fp64 product; the R1 requant of C (the reference's C_out /
    C_scales_row, here [M][N/32]) is bit-exact against the oracle on the GPU's C."""
    M, K, N = 512, 1024, 768
    X = torch.empty((M, K), dtype=torch.float32, device=DEV)
    W = torch.empty((K, N), dtype=torch.float32, device=DEV)
    mxfa.fill_normal(X, 31)
    mxfa.fill_normal(W, 32)
    xq, xs = mxfa.quantize_rows(X)                        # [M][K], [M][K/32]
    wq, ws = mxfa.quantize_cols(W)                        # [K][N], [K/32][N]
    c = mxfa.gemm(xq, xs.t().contiguous(), wq, ws)
    torch.cuda.synchronize()
    ref = np_(X).astype(np.float64) @ np_(W).astype(np.float64)
    assert rel_l2(np_(c), ref) < 0.05
    codes, scales = mxfa.quantize_rows(c)
    oc, osc = O.quantize_rows(np_(c), O.FMT_E4M3)
    np.testing.assert_array_equal(np_(scales), osc)
    np.testing.assert_array_equal(np_(codes), oc)


def test_gemm_bf16_output_is_rne_of_fp32():
    """c_fmt = C_BF16 writes the same accumulators rounded to bf16 (nearest even): bit-equal
    to torch's fp32 -> bf16 conversion of the fp32 output, ragged shapes included."""
    for M, N, K, seed in ((256, 256, 512, 21), (272, 528, 320, 22)):
        rng = np.random.default_rng(seed)
        a, b = _codes(rng, (M, K), 0), _codes(rng, (K, N), 0)
        sa = rng.integers(112, 142, (K // 32, M)).astype(np.uint8)
        sb = rng.integers(112, 142, (K // 32, N)).astype(np.uint8)
        dev = [torch.from_numpy(x).to(DEV) for x in (a, sa, b, sb)]
        c32 = mxfa.gemm(*dev)
        c16 = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
        mxfa.gemm(*dev, out=c16, c_fmt=mxfa.C_BF16)
        torch.cuda.synchronize()
        assert torch.equal(c16.view(torch.int16), c32.to(torch.bfloat16).view(torch.int16))


def test_gemm_deterministic():
    rng = np.random.default_rng(5)
    a, b = _codes(rng, (256, 512), 0), _codes(rng, (512, 256), 0)
    sa = rng.integers(120, 134, (16, 256)).astype(np.uint8)
    sb = rng.integers(120, 134, (16, 256)).astype(np.uint8)
    dev = [torch.from_numpy(x).to(DEV) for x in (a, sa, b, sb)]
    c1 = mxfa.gemm(*dev)
    c2 = mxfa.gemm(*dev)
    torch.cuda.synchronize()
    assert torch.equal(c1, c2)


def test_gemm_benched_shape_sampled():
    """The shape the bench quotes (QKV projection of configs[2]: M 8192, N 6144, K 4096):
    the whole C is computed and checked finite; 96 sampled rows x 96 sampled columns
    (every tile row and column of the 256 x 256 C tiles, and tile edges) against the
    oracle's exact sums, to the same bounds."""
    M, N, K = 8192, 6144, 4096
    print(f"gemm benched shape M{M} N{N} K{K}", flush=True)
    rng = np.random.default_rng(77)
    a, b = _codes(rng, (M, K), mxfa.FMT_E4M3), _codes(rng, (K, N), mxfa.FMT_E4M3)
    sa = rng.integers(112, 142, (K // 32, M)).astype(np.uint8)
    sb = rng.integers(112, 142, (K // 32, N)).astype(np.uint8)
    dev = [torch.from_numpy(x).to(DEV) for x in (a, sa, b, sb)]
    out = mxfa.gemm(dev[0], dev[1], dev[2], dev[3])
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()), "coverage"
    rows = np.unique(np.concatenate([np.arange(0, M, 256), np.arange(255, M, 256)[:32], rng.integers(0, M, 32)]))[:96]
    cols = np.unique(np.concatenate([np.arange(0, N, 256), np.arange(255, N, 256)[:24], rng.integers(0, N, 48)]))[:96]
    c = np_(out)[np.ix_(rows, cols)].astype(np.float64)
    want, ab = O.mx_gemm(np.ascontiguousarray(a[rows]), np.ascontiguousarray(sa[:, rows]),
                         np.ascontiguousarray(b[:, cols]), np.ascontiguousarray(sb[:, cols]),
                         mxfa.FMT_E4M3, mxfa.FMT_E4M3, with_abs=True)
    err = np.abs(c - want)
    print(f"   sampled rel-L2 {rel_l2(c, want):.2e}, max err / sum|terms| {float((err / ab).max()):.2e}", flush=True)
    assert np.all(err <= ab * 2.0 ** -8 + 1e-38)
    assert rel_l2(c, want) <= 1e-3


@pytest.mark.parametrize("M,N,K", [(512, 768, 1024), (272, 528, 512), (8192, 6144, 4096)])
def test_gemm_dma_kernel_equals_register_staged(monkeypatch, M, N, K):
    """E4M3 operands with K % 128 == 0 run the LDS-DMA kernel (unpadded XOR-swizzled tiles); the
    register-staged kernel (MXFA_GEMM=reg) runs the same MFMAs on the same operands in the same
    order, so C must match bit for bit, fp32 and bf16 -- ragged M and N included."""
    rng = np.random.default_rng(M + N + K)
    a, b = _codes(rng, (M, K), 0), _codes(rng, (K, N), 0)
    sa = rng.integers(112, 142, (K // 32, M)).astype(np.uint8)
    sb = rng.integers(112, 142, (K // 32, N)).astype(np.uint8)
    dev = [torch.from_numpy(x).to(DEV) for x in (a, sa, b, sb)]
    for c_fmt, dt in ((mxfa.C_F32, torch.float32), (mxfa.C_BF16, torch.bfloat16)):
        outs = []
        for mode in ("dma", "reg"):
            monkeypatch.setenv("MXFA_GEMM", mode)
            c = torch.full((M, N), float("nan"), dtype=dt, device=DEV)
            mxfa.gemm(*dev, out=c, c_fmt=c_fmt)
            outs.append(c)
        torch.cuda.synchronize()
        assert bool(torch.isfinite(outs[0]).all())
        assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("M,N,K", [(16, 64, 64), (32, 96, 1024), (48, 80, 192), (64, 6144, 4096), (96, 208, 576),
                                   (128, 512, 2048), (112, 48, 4160)])
def test_gemm_skinny_matches_oracle_and_tiled_kernel(monkeypatch, M, N, K):
    """M <= 128 with E4M3 operands runs the skinny kernel (one workgroup per 32-column strip, the
    64-k steps split over its four waves, partials summed in wave order): within the oracle's
    bound like every mxfa_gemm, close to the tiled kernel (MXFA_GEMM=big: the same products,
    accumulated in another order), deterministic, fp32 and bf16 C."""
    print(f"skinny gemm M{M} N{N} K{K}", flush=True)
    rng = np.random.default_rng(M * 7 + N + K)
    a, b = _codes(rng, (M, K), 0), _codes(rng, (K, N), 0)
    sa = rng.integers(112, 142, (K // 32, M)).astype(np.uint8)
    sb = rng.integers(112, 142, (K // 32, N)).astype(np.uint8)
    dev = [torch.from_numpy(x).to(DEV) for x in (a, sa, b, sb)]
    outs = {}
    for mode in ("skinny", "big"):
        if mode == "big":
            monkeypatch.setenv("MXFA_GEMM", "big")
        c = torch.full((M, N), float("nan"), dtype=torch.float32, device=DEV)
        mxfa.gemm(*dev, out=c)
        c16 = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
        mxfa.gemm(*dev, out=c16, c_fmt=mxfa.C_BF16)
        outs[mode] = (c, c16)
    monkeypatch.delenv("MXFA_GEMM")
    c2 = torch.empty((M, N), dtype=torch.float32, device=DEV)
    mxfa.gemm(*dev, out=c2)
    torch.cuda.synchronize()
    c, c16 = outs["skinny"]
    assert torch.equal(c, c2), "not deterministic"
    assert torch.equal(c16.view(torch.int16), c.to(torch.bfloat16).view(torch.int16)), "bf16 C is not the RNE of fp32 C"
    want, ab = O.mx_gemm(a, sa, b, sb, mxfa.FMT_E4M3, mxfa.FMT_E4M3, with_abs=True)
    got = np_(c).astype(np.float64)
    err = np.abs(got - want)
    print(f"   rel-L2 {rel_l2(got, want):.2e}, max err / sum|terms| {float((err / np.maximum(ab, 1e-300)).max()):.2e}",
          flush=True)
    assert np.all(np.isfinite(got))
    assert np.all(err <= ab * 2.0 ** -8 + 1e-38)
    assert rel_l2(got, want) <= 1e-3
    big = np_(outs["big"][0]).astype(np.float64)
    # the same products; the partial sums enter the MFMAs' accumulation in another order
    assert np.all(np.abs(got - big) <= ab * 2.0 ** -12 + 1e-38)
