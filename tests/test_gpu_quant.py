"""GPU parity of the MX quantizers and of the attention kernels' P requant routine:
bit-exact against the oracle (rule R1 of lib/golden, pinned in test_oracle_rules)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import mxfa  # noqa: E402
import oracle as O  # noqa: E402
from gpuhelp import DEV, np_  # noqa: E402

pytestmark = pytest.mark.gpu


def edge_rows(rng):
    """Rows of 32 that stress the scale and element rules."""
    rows = []
    for e in range(-30, 30, 3):
        base = np.float32(2.0 ** e)
        b = np.array(base).view(np.uint32)
        near = (b + np.arange(-16, 16, dtype=np.int64)).astype(np.uint32).view(np.float32)
        rows.append(near)                                            # amax just below / above a power of two
        rows.append(np.float32(2.0 ** e) * (1 + np.arange(32, dtype=np.float32) / 32) * np.where(np.arange(32) % 2, -1, 1))
        r = rng.standard_normal(32).astype(np.float32) * base
        r[0] = base * np.float32(1.999999)                           # block max near the log2f window
        rows.append(r)
        f = np.full(32, base, np.float32) * np.float32(2.0 ** -14) * (np.arange(32, dtype=np.float32) / 16 + 0.5)
        f[0] = base                                                  # flush boundary relative to the max
        rows.append(f)
    rows.append(np.zeros(32, np.float32))
    rows.append(np.full(32, -0.0, np.float32))
    rows.append(np.full(32, 1e-42, np.float32))
    x = np.zeros(32, np.float32); x[3] = np.nan; x[5] = 2.5; rows.append(x)
    x = np.ones(32, np.float32); x[7] = np.inf; rows.append(x)
    x = np.ones(32, np.float32) * 3e38; rows.append(x)
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("fmt", [mxfa.FMT_E4M3, mxfa.FMT_E3M2])
def test_quantize_rows_bit_exact(fmt):
    rng = np.random.default_rng(100 + fmt)
    e = edge_rows(rng)
    e = e[: len(e) // 2 * 2].reshape(-1, 64)
    x = np.concatenate([e, (rng.standard_normal((4096, 64)) * 2.0 ** rng.integers(-20, 20, (4096, 1))).astype(np.float32)])
    xd = torch.from_numpy(np.ascontiguousarray(x)).to(DEV)
    codes, scales = mxfa.quantize_rows(xd, fmt)
    oc, osc = O.quantize_rows(x, fmt)
    np.testing.assert_array_equal(np_(scales), osc)
    bad = np.argwhere(np_(codes) != oc)
    assert len(bad) == 0, [(float(x[i, j]), int(np_(codes)[i, j]), int(oc[i, j])) for i, j in bad[:8]]


@pytest.mark.parametrize("fmt", [mxfa.FMT_E4M3, mxfa.FMT_E3M2])
def test_quantize_cols_bit_exact(fmt):
    rng = np.random.default_rng(200 + fmt)
    x = (rng.standard_normal((3, 128, 96)) * 2.0 ** rng.integers(-8, 8, (3, 1, 96))).astype(np.float32)
    x[0, :32, 5] = 0.0
    x[1, 40, 7] = np.float32(2.0 ** 10) * np.float32(0.99999994)
    xd = torch.from_numpy(x).to(DEV)
    codes, scales = mxfa.quantize_cols(xd, fmt)
    oc, osc = O.quantize_cols(x, fmt)
    np.testing.assert_array_equal(np_(scales), osc)
    np.testing.assert_array_equal(np_(codes), oc)


def test_e3m2_quantizer_covers_all_bf16_magnitudes_below_32():
    """Blocks whose max is 31 have scale code 127 (scale 1.0), so every other element is
    encoded as itself: sweep all bf16 patterns of magnitude < 32, both signs."""
    bits = np.arange(0, 0x4200, dtype=np.uint32)            # bf16 patterns up to 32.0
    vals = (bits << 16).view(np.float32)
    vals = np.concatenate([vals, -vals])
    n = -(-len(vals) // 31) * 31
    vals = np.concatenate([vals, np.zeros(n - len(vals), np.float32)]).reshape(-1, 31)
    x = np.concatenate([np.full((vals.shape[0], 1), 31.0, np.float32), vals], axis=1)
    xd = torch.from_numpy(np.ascontiguousarray(x)).to(DEV)
    codes, scales = mxfa.quantize_rows(xd, mxfa.FMT_E3M2)
    assert np.all(np_(scales) == 127)
    want = np.fromfile(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden", "e3m2_encode.bin"), np.uint8)
    vb = (x.view(np.uint32) >> 16).astype(np.int64)
    np.testing.assert_array_equal(np_(codes), want[vb])


def p_like(rng, rows):
    """fp32 P tiles as the attention kernels produce them: exp2 of non-positive arguments,
    plus zero blocks, subnormals, and values on the flush/saturation/rounding edges."""
    x = np.exp2(-rng.exponential(6.0, (rows, 64))).astype(np.float32)
    x[rng.random(x.shape) < 0.05] = 0.0
    x[::17] = 0.0
    x[5::23, :32] *= np.float32(2.0 ** -130)                   # subnormal blocks
    edge = []
    for e in range(-40, 1):
        m = np.float32(2.0 ** e)
        r = m * np.float32(2.0 ** -14) * (1 + np.arange(64, dtype=np.float32) / 64)
        r[0] = m * np.float32(1.75)                              # saturation region after scaling
        r[1] = m * np.float32(2.0 ** -6) * np.float32(0.9999999)
        r[2] = m * np.float32(1.0 + 1.0 / 16)                    # RNE tie
        r[32] = np.nextafter(m, np.float32(0))                   # block max just below a power of two
        edge.append(r)
    return np.concatenate([x, np.stack(edge)]).astype(np.float32)


def test_requant_p_bit_exact():
    rng = np.random.default_rng(300)
    p = p_like(rng, 8192)
    pd = torch.from_numpy(p).to(DEV)
    codes, scales = mxfa.requant_p(pd)
    oc, osc = O.quantize_rows(p, O.FMT_E4M3)
    np.testing.assert_array_equal(np_(scales), osc)
    bad = np.argwhere(np_(codes) != oc)
    assert len(bad) == 0, [(float(p[i, j]), int(np_(codes)[i, j]), int(oc[i, j])) for i, j in bad[:8]]


def test_fill_normal_statistics():
    x = torch.empty(1 << 22, dtype=torch.float32, device=DEV)
    mxfa.fill_normal(x, 7)
    a = np_(x).astype(np.float64)
    assert abs(a.mean()) < 3e-3 and abs(a.std() - 1.0) < 3e-3
    y = torch.empty(1 << 22, dtype=torch.float32, device=DEV)
    mxfa.fill_normal(y, 7, outlier_p=0.01, outlier_mul=20.0)
    frac = np.mean(np.abs(np_(y) / np.where(a == 0, 1, a) - 20.0) < 1e-3)
    assert 0.008 < frac < 0.012
    z = torch.empty(1 << 10, dtype=torch.float32, device=DEV)
    mxfa.fill_normal(z, 7)
    np.testing.assert_array_equal(np_(z), a[:1 << 10].astype(np.float32))   # counter-based: prefix-stable
