"""A seeded sweep of small attention configurations across the parameter space the entry
points accept: batch, query/KV heads (GQA groups 1-8), ragged query lengths, key lengths
(multiples of 32) with and without a larger kv_stride, query position offsets, causal or not,
sliding windows, softcap, P rules R1 and R2, head dims 64/128/256, V as E4M3, E3M2 bytes or
block-packed E3M2.  Every case runs mxfa_prefill_ws, mxfa_prefill and -- for single-query
cases -- mxfa_decode, each against the oracle at the north_star tolerance (a prefill element
past max-abs must be a traced P code boundary tie, as in test_gpu_attention)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import mxfa  # noqa: E402
import oracle as O  # noqa: E402
from gpuhelp import DEV, MAX_ABS_TOL, REL_L2_TOL, errors, explain_max_abs, np_, oracle_params, sweep_seeds  # noqa: E402

pytestmark = pytest.mark.gpu

FMTS = (mxfa.FMT_E4M3, mxfa.FMT_E3M2, mxfa.FMT_E3M2_BLK)


def _case(i):
    rng = np.random.default_rng(9000 + i)
    D = int(rng.choice([64, 128, 256]))
    Hkv = int(rng.choice([1, 2, 3]))
    group = int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 3))
    Sq = 1 if i % 4 == 3 else int(rng.integers(1, 200))
    Sk = 32 * int(rng.integers(1, 12))
    kv_stride = Sk + 32 * int(rng.integers(0, 3))
    causal = bool(rng.integers(0, 2)) or Sq == 1
    q_pos0 = int(rng.integers(0, Sk)) if causal else 0
    if Sq == 1:
        q_pos0 = Sk - 1 - int(rng.integers(0, 32))
    window = int(rng.choice([0, 0, 40, 100]))
    softcap = float(rng.choice([0.0, 0.0, 20.0, 50.0]))
    p_rule = int(rng.integers(0, 2))
    v_fmt = FMTS[i % 3]
    return dict(B=B, Hq=Hkv * group, Hkv=Hkv, Sq=Sq, Sk=Sk, D=D, kv_stride=kv_stride, causal=causal, q_pos0=q_pos0,
                window=window, softcap=softcap, p_rule=p_rule, v_fmt=v_fmt, seed=9000 + i)


@pytest.mark.parametrize("i", sweep_seeds(list(range(36)) + [286, 292, 812, 2286]))
def test_sweep(i):
    c = _case(i)
    print(f"sweep case {i}: {c}", flush=True)
    B, Hq, Hkv, Sq, Sk, D, L = c["B"], c["Hq"], c["Hkv"], c["Sq"], c["Sk"], c["D"], c["kv_stride"]
    rng = np.random.default_rng(c["seed"])
    Q = rng.standard_normal((B, Hq, Sq, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, L, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, L, D)).astype(np.float32)
    q, qs = mxfa.quantize_rows(torch.from_numpy(Q).to(DEV))
    k, ks = mxfa.quantize_rows(torch.from_numpy(K).to(DEV))
    vbytes_fmt = mxfa.FMT_E4M3 if c["v_fmt"] == mxfa.FMT_E4M3 else mxfa.FMT_E3M2
    v, vs = mxfa.quantize_cols(torch.from_numpy(V).to(DEV), c["v_fmt"])
    kw = dict(causal=c["causal"], q_pos0=c["q_pos0"], window=c["window"], softcap=c["softcap"], p_rule=c["p_rule"])
    p = mxfa.make_params(B, Hq, Hkv, Sq, Sk, D, v_fmt=c["v_fmt"], kv_stride=L, **kw)
    # the oracle on dense copies of the first Sk keys, V codes one per byte
    pe = mxfa.make_params(B, Hq, Hkv, Sq, Sk, D, v_fmt=vbytes_fmt, **kw)
    vh = np_(v)
    if c["v_fmt"] == mxfa.FMT_E3M2_BLK:
        vh = mxfa.e3m2_from_blk(vh)
    cc = np.ascontiguousarray
    oq = (np_(q), np_(qs), cc(np_(k)[:, :, :Sk]), cc(np_(ks)[:, :, :Sk]), cc(vh[:, :, :Sk]),
          cc(np_(vs)[:, :, :Sk // 32]))
    runs = [("prefill_ws", None), ("prefill", False)]
    if Sq == 1:
        runs.append(("decode", "decode"))
    for name, ws in runs:
        if name == "decode":
            out = mxfa.decode(p, q, qs, k, ks, v, vs)
            n_parts, _ = mxfa.decode_plan(p)
            want = O.attention(oracle_params(pe), *oq, block_n=mxfa.DEFAULT_BLOCK_N, n_parts=n_parts)
        else:
            out = mxfa.prefill(p, q, qs, k, ks, v, vs, workspace=ws)
            want = O.attention(oracle_params(pe), *oq, block_n=mxfa.DEFAULT_BLOCK_N)
        torch.cuda.synchronize()
        o = np_(out)
        assert np.all(np.isfinite(o)), name
        rel, mab = errors(o, want)
        print(f"   {name}: rel-L2 {rel:.3e} max-abs {mab:.3e}", flush=True)
        assert rel <= REL_L2_TOL, name
        if mab > MAX_ABS_TOL:
            # only P code boundary ties between the kernel's fp32 and the oracle's double P may
            # exceed the bound (seeds 286, 292, 812 and 2286 of this generator do): traced on dense copies
            # of the first Sk keys, whose O is the strided call's bit for bit
            assert name != "decode", name
            pd = mxfa.make_params(B, Hq, Hkv, Sq, Sk, D, v_fmt=c["v_fmt"], **kw)
            nblk = Sk // 32
            dev = dict(q=q, qs=qs, k=k[:, :, :Sk].contiguous(), ks=ks[:, :, :Sk].contiguous(),
                       v=(v[:, :, :nblk] if c["v_fmt"] == mxfa.FMT_E3M2_BLK else v[:, :, :Sk]).contiguous(),
                       vs=vs[:, :, :nblk].contiguous())
            od = mxfa.prefill(pd, *(dev[n] for n in ("q", "qs", "k", "ks", "v", "vs")), workspace=ws)
            torch.cuda.synchronize()
            assert torch.equal(od, out), "strided and dense calls differ"
            explain_max_abs(pd, dev, {n: np_(x) for n, x in dev.items()}, o, want)
