"""A seeded sweep of medium prefill problems: key lengths 256-5,088, query lengths 33-5,088
(chunked prefill at the cache end, or self-attention), GQA groups 1-8, windows with and
without causal masking, softcap, 1% x20 outliers, P rules R1 and R2, head dims 64/128/256, V
as E4M3, E3M2 bytes or block-packed E3M2.  Every case runs mxfa_prefill_ws and mxfa_prefill
(bit-identical with E4M3 V) and compares two sampled heads with the oracle; a case past
max-abs is compared on every head and each element past the bound must be a traced P code,
scale or flush boundary tie (explain_max_abs).  MXFA_MEDIUM_SEEDS=0-600 runs the exploratory
length of the sweep."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import mxfa  # noqa: E402
import oracle as O  # noqa: E402
from gpuhelp import (MAX_ABS_TOL, REL_L2_TOL, errors, explain_max_abs, gen_qkv, np_, oracle_params,  # noqa: E402
                     sweep_seeds)

pytestmark = pytest.mark.gpu


def _case(i):
    rng = np.random.default_rng(77000 + i)
    D = int(rng.choice([64, 128, 256]))
    Hkv = int(rng.choice([1, 2, 4]))
    group = int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 3))
    Sk = 32 * int(rng.integers(8, 160))
    causal = bool(rng.integers(0, 3))
    Sq = int(rng.integers(33, 1200)) if rng.integers(0, 2) else Sk
    Sq = min(Sq, Sk) if causal else Sq
    q_pos0 = (Sk - Sq) if causal else 0
    window = int(rng.choice([0, 0, 257, 1000]))
    softcap = float(rng.choice([0.0, 0.0, 30.0]))
    v_fmt = int(rng.choice([mxfa.FMT_E4M3, mxfa.FMT_E3M2, mxfa.FMT_E3M2_BLK]))
    p_rule = int(rng.integers(0, 2))
    outlier_p = float(rng.choice([0.0, 0.01]))
    return dict(B=B, Hq=Hkv * group, Hkv=Hkv, Sq=Sq, Sk=Sk, D=D, causal=causal, q_pos0=q_pos0, window=window,
                softcap=softcap, v_fmt=v_fmt, p_rule=p_rule, outlier_p=outlier_p, seed=77000 + i)


@pytest.mark.parametrize("i", sweep_seeds(range(8), "MXFA_MEDIUM_SEEDS"))
def test_medium_sweep(i):
    c = _case(i)
    print(f"medium sweep case {i}: {c}", flush=True)
    B, Hq, Sq, D = c["B"], c["Hq"], c["Sq"], c["D"]
    _, dev, host = gen_qkv(B, Hq, c["Hkv"], Sq, c["Sk"], D, c["seed"], outlier_p=c["outlier_p"], v_fmt=c["v_fmt"])
    p = mxfa.make_params(B, Hq, c["Hkv"], Sq, c["Sk"], D, causal=c["causal"], q_pos0=c["q_pos0"], window=c["window"],
                         softcap=c["softcap"], v_fmt=c["v_fmt"], p_rule=c["p_rule"])
    ops = [dev[n] for n in ("q", "qs", "k", "ks", "v", "vs")]
    o_ws = mxfa.prefill(p, *ops)
    o_nw = mxfa.prefill(p, *ops, workspace=False)
    torch.cuda.synchronize()
    if c["v_fmt"] == mxfa.FMT_E4M3:
        assert torch.equal(o_ws, o_nw), "mxfa_prefill_ws and mxfa_prefill differ"
    # the oracle reads E3M2 V one code per byte
    vh = mxfa.e3m2_from_blk(host["v"]) if c["v_fmt"] == mxfa.FMT_E3M2_BLK else host["v"]
    pe = p
    if c["v_fmt"] == mxfa.FMT_E3M2_BLK:
        pe = type(p).from_buffer_copy(p)
        pe.v_fmt = mxfa.FMT_E3M2
    op = oracle_params(pe)
    nh = B * Hq
    heads = sorted({int(x) for x in np.random.default_rng(i).integers(0, nh, 2)})
    want = O.attention(op, host["q"], host["qs"], host["k"], host["ks"], vh, host["vs"], block_n=mxfa.DEFAULT_BLOCK_N,
                       heads=heads)
    full = None
    for name, out in (("prefill_ws", o_ws), ("prefill", o_nw)):
        o = np_(out)
        assert np.all(np.isfinite(o)), name
        sel = lambda a: a.reshape(nh, Sq, D)[heads]
        rel, mab = errors(sel(o), sel(want))
        print(f"   {name} heads {heads}: rel-L2 {rel:.3e} max-abs {mab:.3e}", flush=True)
        assert rel <= REL_L2_TOL, name
        if mab > MAX_ABS_TOL:
            if full is None:
                full = O.attention(op, host["q"], host["qs"], host["k"], host["ks"], vh, host["vs"],
                                   block_n=mxfa.DEFAULT_BLOCK_N)
            explain_max_abs(p, dev, host, o, full, max_rows=500)
