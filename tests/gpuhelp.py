"""GPU test helpers: synthetic inputs quantized on the GPU (through the C ABI),
copied to the host for the oracle."""
import math

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


def sweep_seeds(default, env="MXFA_SWEEP_SEEDS"):
    """The seeds of a seeded sweep: `default`, or those the environment variable lists
    ("a-b" for a..b-1, comma-separated items), so that a longer exploratory run is one
    pytest command, e.g. MXFA_SWEEP_SEEDS=36-2012."""
    import os
    spec = os.environ.get(env)
    if not spec:
        return list(default)
    out = []
    for item in spec.split(","):
        if "-" in item:
            a, b = item.split("-")
            out += list(range(int(a), int(b)))
        else:
            out.append(int(item))
    return out


REL_L2_TOL = 5e-3     # north_star: rel-L2 <= 5e-3
MAX_ABS_TOL = 2e-2    # north_star: max-abs <= 2e-2


def _decode_table(fmt):
    f = O.lib().orc_e3m2_decode if fmt == "e3m2" else O.lib().orc_e4m3_decode
    return np.array([f(c) for c in range(256)], np.float64)


def _p_block_codes(P, p_rule):
    """Codes and scale of one 32-key block of fp32 P under the P rule (oracle)."""
    import mxfa
    x = np.ascontiguousarray(P, np.float32).reshape(1, -1)
    if p_rule == mxfa.P_R2:
        _, c, s = O.r2_quantize_rows(x)
    else:
        c, s = O.quantize_rows(x, O.FMT_E4M3)
    return c[0], int(s[0, 0])


def _bf16(x):
    """fp32 -> bf16 (round to nearest even), returned as float64."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16).astype(np.uint32)).view(np.float32).astype(np.float64)


def explain_max_abs(p, dev, host, got, want, max_rows=8, rel_tie=2e-5):
    """Account for every O element of a prefill beyond MAX_ABS_TOL.

    The P rule (R1 or R2) maps each P / scale to an E4M3 code; where P lies on the boundary
    between two codes up to the fp32 precision of the kernel's scores and exponential (the
    oracle computes them in double), the two land on adjacent codes, and with a peaked row
    (small l) and a large V element one such code moves O by more than the max-abs bound.
    For each offending row this traces the kernel's own P codes and scales
    (mxfa_prefill_trace) and the oracle's (orc_attention_trace) and asserts: every 32-key
    block whose scales differ is on a scale boundary (scaling the
    block's oracle P by 1 -+ rel_tie gives exactly the two scales, and the kernel's and the
    oracle's codes of the block are the rule's for their scale -- the tile amax next to a
    power of two, e.g. near-saturated softcap scores that are equal in fp32 but not in
    double); outside such blocks at most 4 codes differ, each to an adjacent code (or across R1's
    flush boundary, 0 against the smallest normal); scaling the oracle's P of that
    key by 1 - rel_tie and 1 + rel_tie (its 32-key block otherwise unchanged, the rule
    applied by the oracle) gives exactly those two codes, i.e. P sits on a code boundary;
    and the row's error in every column is within MAX_ABS_TOL of what those code and block
    differences contribute to O (sum of |dequantized difference| * exp(m_block -
    m_final) * |V| / l_final) plus what a differing row sum contributes (|O| |dl| / l).
    Under R2 the row sum adds the bf16-rounded P, so a P on a bf16 rounding boundary moves
    l by one bf16 step of that P: a row sum that differs by more than 1e-4 relative (the
    fp32 sums of R1 stay within a few 1e-6) must be
    covered by the bf16 steps of the row's keys whose bf16 rounding flips between P (1 -
    rel_tie) and P (1 + rel_tie).  Returns the number of rows explained; fails on more than
    max_rows rows."""
    import mxfa
    err = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    bad = np.argwhere(err > MAX_ABS_TOL)
    rows = sorted({(int(b), int(h), int(q)) for b, h, q, _ in bad})
    print(f"   {len(bad)} elements beyond max-abs in {len(rows)} rows", flush=True)
    assert len(rows) <= max_rows, "too many rows beyond max-abs to be rounding ties"
    e4 = _decode_table("e4m3")
    vfmt = "e3m2" if p.v_fmt in (mxfa.FMT_E3M2, mxfa.FMT_E3M2_BLK) else "e4m3"
    vt = _decode_table(vfmt)
    vh = host["v"] if p.v_fmt != mxfa.FMT_E3M2_BLK else mxfa.e3m2_from_blk(host["v"])
    ops = [dev[n] for n in ("q", "qs", "k", "ks", "v", "vs")]
    tp = p
    if p.v_fmt == mxfa.FMT_E3M2_BLK:
        # the stage trace and the oracle read E3M2 V one code per byte: the same codes, and P
        # (what is traced) does not depend on V
        tp = type(p).from_buffer_copy(p)
        tp.v_fmt = mxfa.FMT_E3M2
        ops[4] = torch.from_numpy(np.ascontiguousarray(vh)).to(dev["v"].device)
    op = oracle_params(tp)
    bn = mxfa.DEFAULT_BLOCK_N
    group = p.num_q_heads // p.num_kv_heads
    for b, h, q in rows:
        bh = b * p.num_q_heads + h
        tr = mxfa.prefill_trace(tp, *ops, bh, q // 32)
        ow = O.attention_trace(op, host["q"], host["qs"], host["k"], host["ks"], vh, host["vs"], bn, bh, q)
        r = q % 32
        vis = ~np.isneginf(ow["S"])
        nblk_sc = (np.nonzero(vis)[0].max() // 32) + 1
        ksc, osc = tr["scales"][r][:nblk_sc].astype(int), ow["scales"][:nblk_sc].astype(int)
        sdiff = np.nonzero(ksc != osc)[0]
        kc, oc = tr["codes"][r], ow["codes"]
        in_sblk = np.zeros(len(kc), bool)
        for t in sdiff:
            in_sblk[32 * t:32 * t + 32] = True
        diff = np.nonzero((kc != oc) & ~in_sblk)[0]
        assert len(diff) <= 4, f"row b{b} h{h} q{q}: {len(diff)} codes differ"
        jlast = np.nonzero(vis)[0].max() // bn
        m_f, l_f = ow["m"][jlast], ow["l"][jlast]
        dl = abs(float(tr["l"][jlast, r]) - l_f)
        if dl > 1e-4 * l_f:
            assert p.p_rule == mxfa.P_R2, f"row b{b} h{h} q{q}: row sums differ by {dl / l_f:.2e}"
            keys = np.nonzero(vis)[0]
            m_k = np.asarray(ow["m"])[keys // bn]
            pk = np.exp(ow["S"][keys] - m_k).astype(np.float32)
            step = np.abs(_bf16(pk * np.float32(1.0 + rel_tie)) - _bf16(pk * np.float32(1.0 - rel_tie)))
            ties = step * np.exp(m_k - m_f)
            print(f"   row b{b} h{h} q{q}: row sums differ by {dl:.3e} (l {l_f:.4f}); bf16 ties of the row's P "
                  f"cover {ties.sum():.3e} over {int((ties > 0).sum())} keys", flush=True)
            assert dl <= 1.01 * ties.sum() + 1e-6 * l_f, "the row sums differ beyond the row's bf16 ties"
        assert len(diff) > 0 or len(sdiff) > 0 or dl > 1e-4 * l_f, \
            f"row b{b} h{h} q{q}: neither codes, scales nor row sums differ"
        vrow = vh[b, h // group].astype(np.int64)
        vs = host["vs"][b, h // group].astype(np.int64)
        contrib = np.zeros(p.head_dim)
        # a block whose P scale differs: its amax sits on a scale boundary of the rule (a power
        # of two; under R2 the bf16 rounding of P next to one), so scaling the block's P by
        # 1 -+ rel_tie gives exactly the two scales, and each side's codes are the rule's for
        # that scale; the whole block's requantization difference enters the bound
        for t in sdiff:
            k0 = 32 * t
            m_j = ow["m"][k0 // bn]
            blk = np.where(np.isneginf(ow["S"][k0:k0 + 32]), 0.0, np.exp(ow["S"][k0:k0 + 32] - m_j)).astype(np.float32)
            (clo, slo), (chi, shi) = (_p_block_codes(blk * np.float32(1.0 - rel_tie), p.p_rule),
                                      _p_block_codes(blk * np.float32(1.0 + rel_tie), p.p_rule))
            print(f"   row b{b} h{h} q{q} block {t}: kernel/oracle scales {ksc[t]}/{osc[t]}, amax "
                  f"{float(blk.max()):.7f}; with P x (1 -+ {rel_tie}): {slo}/{shi}", flush=True)
            assert {slo, shi} == {int(ksc[t]), int(osc[t])}, "a differing P scale is not on a scale boundary"
            kside, oside = (clo if slo == ksc[t] else chi), (clo if slo == osc[t] else chi)
            assert np.array_equal(kc[k0:k0 + 32], kside) and np.array_equal(oc[k0:k0 + 32], oside), \
                "a block's codes do not follow its scale"
            for u in range(k0, k0 + 32):
                dp = abs(e4[kc[u]] * 2.0 ** (ksc[t] - 127) - e4[oc[u]] * 2.0 ** (osc[t] - 127)) * math.exp(m_j - m_f)
                if dp:
                    contrib += dp * np.abs(vt[vrow[u]] * 2.0 ** (vs[u // 32] - 127)) / l_f
        for t in diff:
            # adjacent codes, or the flush boundary of R1 (0 and the smallest normal 2^-6)
            assert abs(int(kc[t]) - int(oc[t])) == 1 or {int(kc[t]), int(oc[t])} == {0x00, 0x08}, \
                f"row b{b} h{h} q{q} key {t}: codes {kc[t]:#04x}/{oc[t]:#04x} not adjacent (scale {ow['scales'][t // 32]})"
            sc = int(ow["scales"][t // 32])
            m_j = ow["m"][t // bn]
            k0 = 32 * (t // 32)
            blk = np.where(np.isneginf(ow["S"][k0:k0 + 32]), 0.0,
                           np.exp(ow["S"][k0:k0 + 32] - m_j)).astype(np.float32)
            lo, hi = blk.copy(), blk.copy()
            lo[t - k0] *= np.float32(1.0 - rel_tie)
            hi[t - k0] *= np.float32(1.0 + rel_tie)
            (clo, slo), (chi, shi) = _p_block_codes(lo, p.p_rule), _p_block_codes(hi, p.p_rule)
            print(f"   row b{b} h{h} q{q} key {t}: kernel/oracle codes {kc[t]:#04x}/{oc[t]:#04x}, "
                  f"P/scale {float(blk[t - k0]) * 2.0 ** (127 - sc):.7f}; with P x (1 -+ {rel_tie}): "
                  f"{clo[t - k0]:#04x}/{chi[t - k0]:#04x}", flush=True)
            assert slo == shi == sc, "the perturbation moves the block scale"
            assert {int(clo[t - k0]), int(chi[t - k0])} == {int(kc[t]), int(oc[t])}, \
                "a differing code is not on a code boundary"
            dp = abs(e4[kc[t]] - e4[oc[t]]) * 2.0 ** (sc - 127) * math.exp(m_j - m_f)
            vdeq = vt[vrow[t]] * 2.0 ** (vs[t // 32] - 127)
            contrib += dp * np.abs(vdeq) / l_f
        bound = contrib + np.abs(np.asarray(want, np.float64)[b, h, q]) * 1.01 * dl / l_f + MAX_ABS_TOL
        assert np.all(err[b, h, q] <= bound), "row error exceeds what its boundary cases contribute"
    return len(rows)
