"""A seeded sweep of decode problems: batch 1-3, 1-4 KV heads, query-head groups 1-32, KV
lengths of 32-4,128 tokens read from a cache with a larger kv_stride, the query 0-31 tokens
before the cache end, windows, softcap, P rules R1 and R2, head dims 64/128/256, V as E4M3,
E3M2 bytes or block-packed E3M2, and split plans from 1 partial per head to hundreds
(MXFA_DECODE_WAVES).  Every case runs mxfa_decode against the oracle with the same partials
at the north_star tolerance, and the in-workgroup merge against the combine kernel bit for
bit."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import mxfa  # noqa: E402
import oracle as O  # noqa: E402
from gpuhelp import DEV, MAX_ABS_TOL, REL_L2_TOL, errors, np_, oracle_params, sweep_seeds  # noqa: E402

pytestmark = pytest.mark.gpu

FMTS = (mxfa.FMT_E4M3, mxfa.FMT_E3M2, mxfa.FMT_E3M2_BLK)


def _case(i):
    rng = np.random.default_rng(50000 + i)
    D = int(rng.choice([64, 128, 256]))
    Hkv = int(rng.integers(1, 5))
    group = int(rng.choice([1, 2, 4, 8, 16, 32]))
    B = int(rng.integers(1, 4))
    L = 32 * int(rng.integers(1, 130))
    kv_stride = L + 32 * int(rng.integers(0, 3))
    q_pos0 = L - 1 - int(rng.integers(0, 32))
    window = int(rng.choice([0, 0, 100, 1000]))
    softcap = float(rng.choice([0.0, 0.0, 30.0]))
    p_rule = int(rng.integers(0, 2))
    waves = int(rng.choice([0, 16, 64, 256, 1024, 4096]))     # 0: the library's plan
    return dict(B=B, Hq=Hkv * group, Hkv=Hkv, L=L, kv_stride=kv_stride, D=D, q_pos0=q_pos0, window=window,
                softcap=softcap, p_rule=p_rule, v_fmt=FMTS[i % 3], waves=waves, rng=rng)


@pytest.mark.parametrize("i", sweep_seeds(range(60)))
def test_decode_sweep(i, monkeypatch):
    c = _case(i)
    rng = c.pop("rng")
    print(f"decode sweep case {i}: {c}", flush=True)
    B, Hq, Hkv, L, S, D = c["B"], c["Hq"], c["Hkv"], c["L"], c["kv_stride"], c["D"]
    if c["waves"]:
        monkeypatch.setenv("MXFA_DECODE_WAVES", str(c["waves"]))
    Q = rng.standard_normal((B, Hq, 1, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    q, qs = mxfa.quantize_rows(torch.from_numpy(Q).to(DEV))
    k, ks = mxfa.quantize_rows(torch.from_numpy(K).to(DEV))
    v, vs = mxfa.quantize_cols(torch.from_numpy(V).to(DEV), c["v_fmt"])
    kw = dict(causal=True, q_pos0=c["q_pos0"], window=c["window"], softcap=c["softcap"], p_rule=c["p_rule"])
    p = mxfa.make_params(B, Hq, Hkv, 1, L, D, v_fmt=c["v_fmt"], kv_stride=S, **kw)
    fused = mxfa.decode(p, q, qs, k, ks, v, vs)
    monkeypatch.setenv("MXFA_DECODE_COMBINE", "kernel")
    combined = mxfa.decode(p, q, qs, k, ks, v, vs)
    torch.cuda.synchronize()
    o = np_(fused)
    assert np.all(np.isfinite(o))
    assert torch.equal(fused, combined)
    # the oracle on dense copies of the first L keys, V codes one per byte
    vh = np_(v)
    if c["v_fmt"] == mxfa.FMT_E3M2_BLK:
        vh = mxfa.e3m2_from_blk(vh)
    pe = mxfa.make_params(B, Hq, Hkv, 1, L, D, v_fmt=mxfa.FMT_E4M3 if c["v_fmt"] == mxfa.FMT_E4M3 else mxfa.FMT_E3M2,
                          **kw)
    cc = np.ascontiguousarray
    n_parts, _ = mxfa.decode_plan(p)
    want = O.attention(oracle_params(pe), np_(q), np_(qs), cc(np_(k)[:, :, :L]), cc(np_(ks)[:, :, :L]),
                       cc(vh[:, :, :L]), cc(np_(vs)[:, :, :L // 32]), block_n=mxfa.DEFAULT_BLOCK_N, n_parts=n_parts)
    rel, mab = errors(o, want)
    print(f"   n_parts {n_parts}: rel-L2 {rel:.3e} max-abs {mab:.3e}", flush=True)
    assert rel <= REL_L2_TOL and mab <= MAX_ABS_TOL
