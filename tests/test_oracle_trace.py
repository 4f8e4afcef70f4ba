"""CPU pins of the oracle's stage trace (orc_attention_trace), recomputed independently: scores
from the dequantized operands, the running max and sum of the block recurrence, and the P codes
from the (separately pinned) block quantizers.  The GPU stage test compares the kernel's own
stages with this trace."""
import numpy as np
import pytest

import oracle as O
from mxdata import dequant_rows, normal_inputs, quantize_qkv


def _visible(kpos, qpos, Sk, causal, window):
    ok = kpos < Sk
    if causal:
        ok &= kpos <= qpos
    if window > 0:
        ok &= kpos + window > qpos
    return ok


@pytest.mark.parametrize("softcap,p_rule,causal,window,q_pos0", [
    (0.0, O.P_R1, True, 0, 128),
    (30.0, O.P_R1, True, 100, 128),
    (0.0, O.P_R2, False, 0, 0),
    (30.0, O.P_R2, True, 70, 64),
])
def test_trace_matches_block_recurrence(softcap, p_rule, causal, window, q_pos0):
    B, Hq, Hkv, Sq, Sk, D, bn = 1, 4, 2, 96, 224, 64, 64
    Q, K, V = normal_inputs(B, Hq, Hkv, Sq, Sk, D, seed=31, outlier_p=0.02)
    q, qs, k, ks, v, vs = quantize_qkv(Q, K, V)
    p = O.make_params(B, Hq, Hkv, Sq, Sk, D, causal=causal, q_pos0=q_pos0, window=window, softcap=softcap,
                      p_rule=p_rule)
    scale = p.softmax_scale
    for bh, qi in ((1, 0), (2, 37), (3, 95)):
        tr = O.attention_trace(p, q, qs, k, ks, v, vs, bn, bh, qi)
        h = bh % Hq
        kvh = h // (Hq // Hkv)
        Qd = dequant_rows(q[0, h, qi], qs[0, h, qi], O.FMT_E4M3)
        Kd = dequant_rows(k[0, kvh], ks[0, kvh], O.FMT_E4M3)
        S = (Kd @ Qd) * scale
        if softcap:
            S = softcap * np.tanh(S / softcap)
        vis = _visible(np.arange(Sk), q_pos0 + qi, Sk, causal, window)
        S = np.where(vis, S, -np.inf)
        np.testing.assert_allclose(tr["S"], S, rtol=1e-10, atol=1e-10)
        m, l = -np.inf, 0.0
        for j in range((Sk + bn - 1) // bn):
            blk = S[j * bn:(j + 1) * bn]
            m_new = max(m, blk.max())
            if m_new == -np.inf:
                assert tr["m"][j] == -np.inf and tr["l"][j] == 0.0
                assert not tr["codes"][j * bn:(j + 1) * bn].any()
                continue
            P = np.where(np.isinf(blk), 0.0, np.exp(blk - m_new)).astype(np.float32)
            if p_rule == O.P_R2:
                P, pc, ps = O.r2_quantize_rows(P.reshape(-1, 32))
            else:
                pc, ps = O.quantize_rows(P.reshape(-1, 32), O.FMT_E4M3)
            corr = 0.0 if m == -np.inf else np.exp(m - m_new)
            l = l * corr + P.astype(np.float64).sum()
            m = m_new
            # numpy's tanh may differ from libm's in the last bit of a double
            np.testing.assert_allclose(tr["m"][j], m, rtol=1e-14)
            np.testing.assert_allclose(tr["l"][j], l, rtol=1e-12)
            np.testing.assert_array_equal(tr["codes"][j * bn:(j + 1) * bn], pc.reshape(-1))
            np.testing.assert_array_equal(tr["scales"][j * bn // 32:(j + 1) * bn // 32], ps.reshape(-1))


def test_trace_rejects_bad_rows():
    Q, K, V = normal_inputs(1, 2, 2, 32, 64, 64, seed=3)
    q, qs, k, ks, v, vs = quantize_qkv(Q, K, V)
    p = O.make_params(1, 2, 2, 32, 64, 64)
    with pytest.raises(ValueError):
        O.attention_trace(p, q, qs, k, ks, v, vs, 64, 2, 0)
    with pytest.raises(ValueError):
        O.attention_trace(p, q, qs, k, ks, v, vs, 64, 0, 32)
