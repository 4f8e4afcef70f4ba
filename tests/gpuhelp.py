"""GPU test helpers: synthetic inputs quantized on the GPU (through the C ABI),
copied to the host for the oracle."""
import numpy as np
import torch

import mxfa
import oracle as O

DEV = "cuda:0"


def np_(t):
    return t.detach().cpu().numpy()


def gen_qkv(B, Hq, Hkv, Sq, Sk, D, seed, outlier_p=0.0, q_mul=1.0, v_fmt=mxfa.FMT_E4M3):
    """fp32 N(0,1) inputs generated on the GPU, quantized on the GPU.  Returns
    (fp32 host arrays, device codes dict, host codes dict)."""
    Q = torch.empty((B, Hq, Sq, D), dtype=torch.float32, device=DEV)
    K = torch.empty((B, Hkv, Sk, D), dtype=torch.float32, device=DEV)
    V = torch.empty((B, Hkv, Sk, D), dtype=torch.float32, device=DEV)
    mxfa.fill_normal(Q, seed * 3 + 1, outlier_p)
    mxfa.fill_normal(K, seed * 3 + 2, outlier_p)
    mxfa.fill_normal(V, seed * 3 + 3, outlier_p)
    if q_mul != 1.0:
        Q.mul_(q_mul)
    q, qs = mxfa.quantize_rows(Q, mxfa.FMT_E4M3)
    k, ks = mxfa.quantize_rows(K, mxfa.FMT_E4M3)
    v, vs = mxfa.quantize_cols(V, v_fmt)
    dev = dict(q=q, qs=qs, k=k, ks=ks, v=v, vs=vs)
    host = {n: np_(t) for n, t in dev.items()}
    return dict(Q=Q, K=K, V=V), dev, host


def oracle_params(p):
    return O.make_params(p.batch, p.num_q_heads, p.num_kv_heads, p.seq_q, p.seq_k, p.head_dim,
                         causal=bool(p.causal), q_pos0=p.q_pos0, window=p.window, scale=p.softmax_scale,
                         softcap=p.softcap, v_fmt=p.v_fmt, p_rule=p.p_rule)


def errors(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    rel = float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))
    mab = float(np.max(np.abs(got - want))) if got.size else 0.0
    return rel, mab


REL_L2_TOL = 5e-3     # north_star: rel-L2 <= 5e-3
MAX_ABS_TOL = 2e-2    # north_star: max-abs <= 2e-2
