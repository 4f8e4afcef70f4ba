"""CPU tests pinning the oracle's streaming MX attention
(kernels/flash_attention_mx_gemma/flash_attention_model.py:317-372 semantics)
with closed forms and invariants rather than a second copy of the recurrence."""
import numpy as np
import pytest

import oracle as O
from mxdata import dequant_cols, dequant_rows, normal_inputs, quantize_qkv, rel_l2


def _single_block_closed_form(q, qs, k, ks, v, vs, scale, mask=None, softcap=0.0, p_rule=O.P_R1):
    """One key block: O = sum_k Pq_k V_k / sum_k P_k with P = fp32(exp(S - max S)) and
    Pq the R1 requant of P per 32 keys (quantizer pinned separately); with rule R2, P is
    first rounded to bf16 and requantized by R2 (pinned separately)."""
    Qd = dequant_rows(q, qs, O.FMT_E4M3)
    Kd = dequant_rows(k, ks, O.FMT_E4M3)
    Vd = dequant_cols(v, vs, O.FMT_E4M3)
    S = (Qd @ Kd.T) * scale
    if softcap:
        S = softcap * np.tanh(S / softcap)
    if mask is not None:
        S = np.where(mask, -np.inf, S)
    m = S.max(axis=1, keepdims=True)
    P = np.where(np.isinf(S), 0.0, np.exp(S - m)).astype(np.float32)
    if p_rule == O.P_R2:
        P, pc, ps = O.r2_quantize_rows(P)
        Pq = dequant_rows(pc, ps, O.FMT_E4M3)
        return (Pq @ Vd) / P.astype(np.float64).sum(axis=1, keepdims=True)
    pc, ps = O.quantize_rows(P, O.FMT_E4M3)
    Pq = dequant_rows(pc, ps, O.FMT_E4M3)
    return (Pq @ Vd) / P.astype(np.float64).sum(axis=1, keepdims=True)


@pytest.mark.parametrize("causal", [False, True])
def test_single_block_closed_form(causal):
    B, H, S, D = 1, 1, 96, 64
    Q, K, V = normal_inputs(B, H, H, S, S, D, seed=3)
    q, qs, k, ks, v, vs = quantize_qkv(Q, K, V)
    p = O.make_params(B, H, H, S, S, D, causal=causal)
    o = O.attention(p, q, qs, k, ks, v, vs, block_n=128)
    mask = np.triu(np.ones((S, S), bool), 1) if causal else None
    want = _single_block_closed_form(q[0, 0], qs[0, 0], k[0, 0], ks[0, 0], v[0, 0], vs[0, 0], p.softmax_scale, mask)
    np.testing.assert_allclose(o[0, 0], want, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("causal", [False, True])
def test_single_block_closed_form_r2(causal):
    """Rule R2 (the reference device kernels' truncating requant of bf16 P) in the
    recurrence: P rounded to bf16 for both the PV codes and the row sum."""
    B, H, S, D = 1, 1, 96, 64
    Q, K, V = normal_inputs(B, H, H, S, S, D, seed=13)
    q, qs, k, ks, v, vs = quantize_qkv(Q, K, V)
    p = O.make_params(B, H, H, S, S, D, causal=causal, p_rule=O.P_R2)
    o = O.attention(p, q, qs, k, ks, v, vs, block_n=128)
    mask = np.triu(np.ones((S, S), bool), 1) if causal else None
    want = _single_block_closed_form(q[0, 0], qs[0, 0], k[0, 0], ks[0, 0], v[0, 0], vs[0, 0], p.softmax_scale, mask,
                                     p_rule=O.P_R2)
    np.testing.assert_allclose(o[0, 0], want, rtol=1e-6, atol=1e-7)
    # truncation only lowers P codes: R2 differs from R1 by at most the 2^-3 relative
    # truncation step of each P, and it is not the R1 result
    o1 = O.attention(O.make_params(B, H, H, S, S, D, causal=causal), q, qs, k, ks, v, vs, block_n=128)
    dense = O.attention_dense(O.make_params(B, H, H, S, S, D, causal=causal), q, qs, k, ks, v, vs)
    assert not np.array_equal(o, o1)
    assert rel_l2(o, dense) < 0.15 and rel_l2(o1, dense) < rel_l2(o, dense)


def test_blocking_exact_when_max_in_first_key():
    """With the row max in key 0 (block 0) corr == 1 for every later block, so any block
    size gives the same P, codes and sums as one block."""
    B, H, S, D = 1, 2, 64, 64
    Q, K, V = normal_inputs(B, H, H, S, 256, D, seed=4)
    Q[..., 0] = 2.0
    K[..., 0] = 0.0
    K[:, :, 0, 0] = 60.0
    q, qs, k, ks, v, vs = quantize_qkv(Q, K, V)
    p = O.make_params(B, H, H, S, 256, D, scale=0.05)
    ref = O.attention(p, q, qs, k, ks, v, vs, block_n=256)
    for bn in (32, 64, 128):
        o = O.attention(p, q, qs, k, ks, v, vs, block_n=bn)
        np.testing.assert_allclose(o, ref, rtol=1e-9, atol=1e-12)
    # split-KV: every split holds a copy of the dominating key, so each split's running
    # max equals the global max and the log-sum-exp merge must reproduce one pass
    K[:, :, 128] = K[:, :, 0]
    q, qs, k, ks, v, vs = quantize_qkv(Q, K, V)
    ref = O.attention(p, q, qs, k, ks, v, vs, block_n=256)
    o = O.attention(p, q, qs, k, ks, v, vs, block_n=64, split_len=128)
    np.testing.assert_allclose(o, ref, rtol=1e-9, atol=1e-12)
    # interleaved partials (partial i = blocks i, i + n, ...): with copies of the dominating
    # key at the start of blocks 0 and 1, both partials of n = 2 see the global max first
    K[:, :, 64] = K[:, :, 0]
    q, qs, k, ks, v, vs = quantize_qkv(Q, K, V)
    ref = O.attention(p, q, qs, k, ks, v, vs, block_n=256)
    o = O.attention(p, q, qs, k, ks, v, vs, block_n=64, n_parts=2)
    np.testing.assert_allclose(o, ref, rtol=1e-9, atol=1e-12)


def test_streaming_close_to_dense_and_fp32():
    """MX flash attention vs unquantized attention: the reference reports ~3.6% (bf16)
    to ~6% Frobenius error; fp32 P with R1 requant stays within 6%."""
    B, Hq, Hkv, S, D = 1, 4, 2, 256, 64
    Q, K, V = normal_inputs(B, Hq, Hkv, S, S, D, seed=5)
    q, qs, k, ks, v, vs = quantize_qkv(Q, K, V)
    p = O.make_params(B, Hq, Hkv, S, S, D, causal=True)
    o = O.attention(p, q, qs, k, ks, v, vs, block_n=64)
    od = O.attention_dense(p, q, qs, k, ks, v, vs)
    assert rel_l2(o, od) < 0.06
    # fp32 reference on the unquantized inputs (torch.softmax semantics)
    Kr = np.repeat(K, Hq // Hkv, axis=1).astype(np.float64)
    Vr = np.repeat(V, Hq // Hkv, axis=1).astype(np.float64)
    Sc = Q.astype(np.float64) @ np.swapaxes(Kr, -1, -2) / np.sqrt(D)
    Sc = np.where(np.triu(np.ones((S, S), bool), 1), -np.inf, Sc)
    P = np.exp(Sc - Sc.max(-1, keepdims=True))
    of = (P / P.sum(-1, keepdims=True)) @ Vr
    assert rel_l2(o, of) < 0.08


def test_gqa_equals_replicated_kv():
    B, Hq, Hkv, S, D = 2, 4, 2, 64, 64
    Q, K, V = normal_inputs(B, Hq, Hkv, S, S, D, seed=6)
    q, qs, k, ks, v, vs = quantize_qkv(Q, K, V)
    p = O.make_params(B, Hq, Hkv, S, S, D, causal=True)
    o = O.attention(p, q, qs, k, ks, v, vs, block_n=32)
    rep = lambda a: np.repeat(a, Hq // Hkv, axis=1)
    p2 = O.make_params(B, Hq, Hq, S, S, D, causal=True)
    o2 = O.attention(p2, q, qs, rep(k), rep(ks), rep(v), rep(vs), block_n=32)
    np.testing.assert_array_equal(o, o2)


def test_causal_and_window_locality():
    """Rows only depend on visible keys: perturbing invisible keys leaves them unchanged."""
    B, H, S, D, W = 1, 1, 128, 64, 40
    Q, K, V = normal_inputs(B, H, H, S, S, D, seed=7)
    p = O.make_params(B, H, H, S, S, D, causal=True, window=W)
    o = O.attention(p, *quantize_qkv(Q, K, V), block_n=32)
    K2, V2 = K.copy(), V.copy()
    rng = np.random.default_rng(8)
    i = 70          # row 70 sees keys 31..70
    K2[:, :, 71:] = rng.standard_normal(K2[:, :, 71:].shape)
    K2[:, :, :31] = rng.standard_normal(K2[:, :, :31].shape)
    V2[:, :, 96:] = rng.standard_normal(V2[:, :, 96:].shape)
    # V is blocked along keys in 32s: leave the blocks containing visible keys untouched
    o2 = O.attention(p, *quantize_qkv(Q, K2, V2), block_n=32)
    np.testing.assert_array_equal(o[0, 0, i], o2[0, 0, i])
    assert not np.array_equal(o[0, 0, 100], o2[0, 0, 100])


def test_fully_masked_rows_are_zero():
    """Reference gemma finalize writes 0 when l <= 0 (flash_mx_impl.hpp:545-560)."""
    B, H, Sq, Sk, D = 1, 1, 32, 64, 32
    Q, K, V = normal_inputs(B, H, H, Sq, Sk, D, seed=9)
    p = O.make_params(B, H, H, Sq, Sk, D, causal=True, q_pos0=200, window=100)
    o = O.attention(p, *quantize_qkv(Q, K, V), block_n=32)
    assert np.all(o == 0.0)


def test_softcap_limits():
    """cap -> infinity is the uncapped recurrence."""
    B, H, S, D = 1, 2, 64, 64
    Q, K, V = normal_inputs(B, H, H, S, S, D, seed=10)
    ops = quantize_qkv(Q, K, V)
    p0 = O.make_params(B, H, H, S, S, D, causal=True)
    pbig = O.make_params(B, H, H, S, S, D, causal=True, softcap=1e12)
    np.testing.assert_allclose(O.attention(pbig, *ops, block_n=32), O.attention(p0, *ops, block_n=32), rtol=1e-6, atol=1e-7)


def _saturated_softcap_case(cap):
    """Scores of exactly +-A (A = 32) after the softmax scale: Q row e0 * 16, K rows
    +-16 e0 (powers of two, exact in E4M3), scale 1/8.  Keys k % 4 == 0 are '+', so
    every 32-key P tile holds a '+' key and its amax is exactly 1.  V is 1.0 on '+'
    keys and 3.0 on '-' keys (exact E4M3 after the along-keys quantization)."""
    B, H, Sq, Sk, D = 1, 1, 4, 64, 64
    Q = np.zeros((B, H, Sq, D), np.float32)
    Q[..., 0] = 16.0
    plus = (np.arange(Sk) % 4) == 0
    K = np.zeros((B, H, Sk, D), np.float32)
    K[0, 0, :, 0] = np.where(plus, 16.0, -16.0)
    V = np.where(plus[:, None], 1.0, 3.0).astype(np.float32)[None, None].repeat(1, 0)
    V = np.broadcast_to(V, (B, H, Sk, D)).copy()
    ops = quantize_qkv(Q, K, V)
    p = O.make_params(B, H, H, Sq, Sk, D, scale=0.125, softcap=cap)
    return p, ops, int(plus.sum()), int((~plus).sum())


def _e4m3_rne(y):
    """Round a positive value in the E4M3 normal range to 3 mantissa bits, ties to even."""
    e = np.floor(np.log2(y))
    m = y / 2.0 ** e * 8.0
    r = np.floor(m)
    frac = m - r
    r = r + (1.0 if frac > 0.5 or (frac == 0.5 and r % 2 == 1) else 0.0)
    return r / 8.0 * 2.0 ** e


@pytest.mark.parametrize("cap", [2.0, 3.0])
def test_softcap_saturation_identity(cap):
    """Gemma order (kernels/flash_attention_mx_gemma/flash_attention_model.py:263-267,
    299-314): s <- cap * tanh((q.k) * scale / cap), then max and exp.  With scaled scores
    +-32 the capped scores are +-cap*tanh(32/cap), so '+' keys weigh 1 and '-' keys
    P = exp(-2 cap tanh(32/cap)); P sits in a tile of amax 1, so its R1 code is the E4M3
    rounding of 256 P at scale 2^-8.  O = (n+ + 3 n- Pq) / (n+ + n- P) in every column.
    Capping before the scale would give P = exp(-2 cap scale) and no cap at all P = 0."""
    p, ops, npl, nmi = _saturated_softcap_case(cap)
    o = O.attention(p, *ops, block_n=64)
    P = float(np.float32(np.exp(-2.0 * cap * np.tanh(32.0 / cap))))
    Pq = _e4m3_rne(256.0 * P) / 256.0
    want = (npl + 3.0 * nmi * Pq) / (npl + nmi * P)
    np.testing.assert_allclose(o, want, rtol=2e-7)
    # the orders this test is meant to reject
    P_swapped = float(np.float32(np.exp(-2.0 * cap * 0.125)))
    Pq_swapped = _e4m3_rne(256.0 * P_swapped) / 256.0
    swapped = (npl + 3.0 * nmi * Pq_swapped) / (npl + nmi * P_swapped)
    assert abs(swapped - want) > 0.2 and abs(1.0 - want) > 1e-3
    # and the oracle streaming over 32-key blocks gives the same (every tile has amax 1)
    np.testing.assert_allclose(O.attention(p, *ops, block_n=32), want, rtol=2e-7)


@pytest.mark.parametrize("cap", [2.0, 50.0])
def test_softcap_closed_form_stressed_window(cap):
    """The reference's softcap stress (Q x 50, kernels/flash_attention_mx_gemma/fa_gen_data.py:
    77-79,98) under a causal sliding window, one key block: the oracle equals the dense
    closed form scale -> cap*tanh(./cap) -> mask -> exp(S - max) -> R1 requant of P ->
    PV / sum P.  With cap 2 every visible score lies in [-2, 2] (weights within e^-4 of the
    max, far from the uncapped result); with cap 50 the stressed scores reach the
    saturating part of tanh."""
    B, H, S, D, W = 1, 1, 96, 64, 40
    Q, K, V = normal_inputs(B, H, H, S, S, D, seed=31, q_mul=50.0)
    ops = quantize_qkv(Q, K, V)
    p = O.make_params(B, H, H, S, S, D, causal=True, window=W, softcap=cap)
    o = O.attention(p, *ops, block_n=128)
    qpos = np.arange(S)[:, None]
    kpos = np.arange(S)[None, :]
    mask = (kpos > qpos) | (kpos + W <= qpos)
    want = _single_block_closed_form(*(a[0, 0] for a in ops), p.softmax_scale, mask, softcap=cap)
    np.testing.assert_allclose(o[0, 0], want, rtol=1e-6, atol=1e-7)
    uncapped = _single_block_closed_form(*(a[0, 0] for a in ops), p.softmax_scale, mask)
    assert rel_l2(o[0, 0], uncapped) > (0.5 if cap == 2.0 else 1e-3)
    if cap == 50.0:
        # the stressed scores do reach the cap: some |scaled score| exceeds cap
        Qd = dequant_rows(ops[0][0, 0], ops[1][0, 0], O.FMT_E4M3)
        Kd = dequant_rows(ops[2][0, 0], ops[3][0, 0], O.FMT_E4M3)
        assert np.abs(Qd @ Kd.T * p.softmax_scale).max() > cap


def test_window_and_causal_edges_exact():
    """Visible keys of row qpos are qpos - W + 1 .. qpos (the reference masks kpos + W <= qpos
    and kpos > qpos, kernels/flash_attention_mx_gemma/flash_attention_model.py:288-296).
    Perturbing the K row of each edge key tells visible from masked: keys qpos - W + 1 and
    qpos change the row, keys qpos - W and qpos + 1 leave it bit-identical (K is blocked
    along D, so one key's K row touches no other key's codes)."""
    B, H, S, D, W = 1, 1, 128, 64, 40
    Q, K, V = normal_inputs(B, H, H, S, S, D, seed=17)
    p = O.make_params(B, H, H, S, S, D, causal=True, window=W)
    base = O.attention(p, *quantize_qkv(Q, K, V), block_n=32)
    rng = np.random.default_rng(18)
    for qpos in (70, 100):
        for key, visible in ((qpos - W + 1, True), (qpos, True), (qpos - W, False), (qpos + 1, False)):
            K2 = K.copy()
            K2[0, 0, key] = rng.standard_normal(D).astype(np.float32) * 3.0
            o2 = O.attention(p, *quantize_qkv(Q, K2, V), block_n=32)
            same = np.array_equal(base[0, 0, qpos], o2[0, 0, qpos])
            assert same != visible, (qpos, key, visible)


def test_split_kv_close_to_single_pass():
    """P is requantized relative to each split's running max, so a different schedule moves
    O by about the MX quantization error itself (~3%): parity tests must run the oracle with
    the kernel's block and split sizes."""
    B, Hq, Hkv, Sk, D = 4, 8, 2, 1024, 128
    Q, K, V = normal_inputs(B, Hq, Hkv, 1, Sk, D, seed=12)
    ops = quantize_qkv(Q, K, V)
    p = O.make_params(B, Hq, Hkv, 1, Sk, D, causal=True, q_pos0=Sk - 1)
    a = O.attention(p, *ops, block_n=64)
    b = O.attention(p, *ops, block_n=64, split_len=256)
    d = O.attention_dense(p, *ops)
    assert rel_l2(b, a) < 0.06 and rel_l2(b, d) < 0.06


def test_interleaved_partials_schedule():
    """n_parts = 1 is the single pass bit for bit; n_parts = number of blocks makes every
    block its own partial, which equals contiguous chunks of one block (split_len =
    block_n) bit for bit; other n_parts differ from the single pass by about the MX
    quantization error.  A schedule that merged partials out of order or took the
    blocks contiguously would fail the identities below."""
    B, Hq, Hkv, Sk, D = 2, 8, 2, 512, 64
    Q, K, V = normal_inputs(B, Hq, Hkv, 1, Sk, D, seed=21)
    ops = quantize_qkv(Q, K, V)
    p = O.make_params(B, Hq, Hkv, 1, Sk, D, causal=True, q_pos0=Sk - 1)
    one = O.attention(p, *ops, block_n=64)
    np.testing.assert_array_equal(O.attention(p, *ops, block_n=64, n_parts=1), one)
    np.testing.assert_array_equal(O.attention(p, *ops, block_n=64, n_parts=8),
                                  O.attention(p, *ops, block_n=64, split_len=64))
    four = O.attention(p, *ops, block_n=64, n_parts=4)
    assert 0 < rel_l2(four, one) < 0.06
    assert not np.array_equal(four, O.attention(p, *ops, block_n=64, split_len=128))
    # partial i of n = 2 over a cache whose odd blocks are all masked (window) equals one
    # pass over the even blocks: here the window keeps only the last block (7, odd), so
    # n = 2 leaves partial 0 empty and equals the single pass
    pw = O.make_params(B, Hq, Hkv, 1, Sk, D, causal=True, q_pos0=Sk - 1, window=64)
    np.testing.assert_array_equal(O.attention(pw, *ops, block_n=64, n_parts=2), O.attention(pw, *ops, block_n=64))


def test_e3m2_v_operand():
    B, Hq, Hkv, S, D = 1, 2, 1, 64, 64
    Q, K, V = normal_inputs(B, Hq, Hkv, S, S, D, seed=13)
    ops = quantize_qkv(Q, K, V, v_fmt=O.FMT_E3M2)
    assert ops[4].max() < 64
    p = O.make_params(B, Hq, Hkv, S, S, D, causal=True, v_fmt=O.FMT_E3M2)
    o = O.attention(p, *ops, block_n=32)
    od = O.attention_dense(p, *ops)
    assert rel_l2(o, od) < 0.06


def test_invalid_arguments_rejected():
    p = O.make_params(1, 3, 2, 32, 32, 64)
    z = np.zeros(1 << 16, np.uint8)
    with pytest.raises(ValueError):
        O.attention(p, z, z, z, z, z, z, block_n=32)
    p = O.make_params(1, 1, 1, 32, 32, 48)
    with pytest.raises(ValueError):
        O.attention(p, z, z, z, z, z, z, block_n=32)
