"""GPU parity of block-packed E3M2 V (FMT_E3M2_BLK: each column's 32-row MX block as 24
bytes of 6-bit codes in the key order of the scaled MFMA's fp6 operand).  The quantizer and the KV-cache append
must give exactly the oracle's E3M2 codes, packed; the prefill kernels, which copy that V
into LDS as it is, must match the oracle to the north_star tolerance and the byte-E3M2 path
to within a few ulps (same values and scales, so the same O up to MFMA summation order)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import mxfa  # noqa: E402
import oracle as O  # noqa: E402
from gpuhelp import DEV, MAX_ABS_TOL, REL_L2_TOL, errors, gen_qkv, np_, oracle_params  # noqa: E402

pytestmark = pytest.mark.gpu

BLK = mxfa.FMT_E3M2_BLK


@pytest.mark.parametrize("shape", [(3, 128, 96), (2, 64, 100)])
def test_quantize_cols_blk_bit_exact(shape):
    rng = np.random.default_rng(610 + shape[2])
    x = (rng.standard_normal(shape) * 2.0 ** rng.integers(-8, 8, (shape[0], 1, shape[2]))).astype(np.float32)
    x[0, :32, 5] = 0.0                                               # an all-zero block
    x[1, 40, 7] = np.float32(2.0 ** 10) * np.float32(0.99999994)      # rounds up to the next binade
    codes, scales = mxfa.quantize_cols(torch.from_numpy(x).to(DEV), BLK)
    oc, osc = O.quantize_cols(x, O.FMT_E3M2)
    assert tuple(codes.shape) == (shape[0], shape[1] // 32, shape[2], 24)
    np.testing.assert_array_equal(np_(scales), osc)
    np.testing.assert_array_equal(np_(codes), mxfa.e3m2_to_blk(oc))


def _e3m2_params(p):
    q = mxfa.make_params(p.batch, p.num_q_heads, p.num_kv_heads, p.seq_q, p.seq_k, p.head_dim, causal=p.causal,
                         q_pos0=p.q_pos0, window=p.window, scale=p.softmax_scale, softcap=p.softcap,
                         v_fmt=mxfa.FMT_E3M2, p_rule=p.p_rule, kv_stride=p.kv_stride)
    return q


def run_blk(B, Hq, Hkv, Sq, Sk, D, seed, heads=None, check_codes=True, outlier_p=0.0, q_mul=1.0, **kw):
    print(f"blk case B{B} Hq{Hq} Hkv{Hkv} Sq{Sq} Sk{Sk} D{D} {kw} seed {seed}", flush=True)
    fp, dev, host = gen_qkv(B, Hq, Hkv, Sq, Sk, D, seed, outlier_p=outlier_p, q_mul=q_mul, v_fmt=mxfa.FMT_E3M2)
    vb, vbs = mxfa.quantize_cols(fp["V"], BLK)
    torch.cuda.synchronize()
    assert torch.equal(vbs, dev["vs"])
    if check_codes:
        np.testing.assert_array_equal(np_(vb), mxfa.e3m2_to_blk(host["v"]))
    p = mxfa.make_params(B, Hq, Hkv, Sq, Sk, D, v_fmt=BLK, **kw)
    pe = _e3m2_params(p)
    want = O.attention(oracle_params(pe), host["q"], host["qs"], host["k"], host["ks"], host["v"], host["vs"],
                       block_n=mxfa.DEFAULT_BLOCK_N, heads=heads)
    sel = (lambda a: a) if heads is None else (lambda a: a.reshape(B * Hq, Sq, D)[np.array(heads)])
    want = sel(want)
    outs = {}
    for ws in (None, False):
        name = "workspace" if ws is None else "workspace-free"
        out = torch.full((B, Hq, Sq, D), float("nan"), dtype=torch.float32, device=DEV)
        mxfa.prefill(p, dev["q"], dev["qs"], dev["k"], dev["ks"], vb, vbs, out=out, workspace=ws)
        ref = mxfa.prefill(pe, dev["q"], dev["qs"], dev["k"], dev["ks"], dev["v"], dev["vs"], workspace=ws)
        torch.cuda.synchronize()
        o = np_(out)
        assert np.all(np.isfinite(o)), f"{name}: some O elements were not written"
        rel, mab = errors(sel(o), want)
        drel, dmab = errors(o, np_(ref))
        print(f"   {name}: rel-L2 {rel:.3e} max-abs {mab:.3e} vs oracle; vs byte E3M2 rel-L2 {drel:.2e} "
              f"max-abs {dmab:.2e} (bit-identical: {torch.equal(out, ref)})", flush=True)
        assert rel <= REL_L2_TOL and mab <= MAX_ABS_TOL
        # the same MX values, so the same O up to summation order inside the MFMA
        assert drel <= 1e-5 and dmab <= 1e-4
        outs[name] = out
    return p, dev, vb, vbs, outs


@pytest.mark.parametrize("case", [
    dict(B=1, Hq=2, Hkv=2, Sq=96, Sk=160, D=64, seed=620),
    dict(B=2, Hq=8, Hkv=2, Sq=200, Sk=320, D=128, seed=621, causal=True, q_pos0=120),
    dict(B=1, Hq=4, Hkv=2, Sq=384, Sk=384, D=256, seed=622, causal=True, window=128, softcap=50.0),
    dict(B=1, Hq=4, Hkv=1, Sq=256, Sk=256, D=128, seed=623, causal=True, softcap=30.0, p_rule=mxfa.P_R2),
    dict(B=1, Hq=2, Hkv=2, Sq=64, Sk=256, D=256, seed=624, causal=True, q_pos0=192, p_rule=mxfa.P_R2),
    dict(B=1, Hq=4, Hkv=4, Sq=128, Sk=128, D=64, seed=625, softcap=50.0, outlier_p=0.01),
])
def test_prefill_blk_matches_oracle(case):
    case = dict(case)
    run_blk(case.pop("B"), case.pop("Hq"), case.pop("Hkv"), case.pop("Sq"), case.pop("Sk"), case.pop("D"),
            case.pop("seed"), outlier_p=case.pop("outlier_p", 0.0), **case)


def test_prefill_blk_config4_shape():
    """The Gemma config at full shape with V block-packed (B=1 Hq=16 Hkv=8 S=8192 D=256,
    window 4096, softcap 50): every head against the oracle."""
    run_blk(1, 16, 8, 8192, 8192, 256, 626, check_codes=False, causal=True, window=4096, softcap=50.0)


@pytest.mark.parametrize("D", [64, 256])
def test_prefill_blk_on_strided_cache(D):
    """kv_stride > seq_k: V blocks past seq_k / 32 hold garbage and are never read; O equals
    the dense call's bit for bit, with and without the workspace."""
    B, Hq, Hkv, Sq, Sk, Lcap = 2, 4, 2, 96, 160, 256
    rng = np.random.default_rng(630 + D)
    mk = lambda *s: torch.from_numpy(rng.standard_normal(s).astype(np.float32)).to(DEV)  # noqa: E731
    q, qs = mxfa.quantize_rows(mk(B, Hq, Sq, D))
    k, ks = mxfa.quantize_rows(mk(B, Hkv, Sk, D))
    v, vs = mxfa.quantize_cols(mk(B, Hkv, Sk, D), BLK)
    garbage = lambda shape: torch.from_numpy(rng.integers(0, 256, shape, dtype=np.uint8)).to(DEV)  # noqa: E731
    kc, ksc = garbage((B, Hkv, Lcap, D)), garbage((B, Hkv, Lcap, D // 32))
    vc, vsc = garbage((B, Hkv, Lcap // 32, D, 24)), garbage((B, Hkv, Lcap // 32, D))
    kc[:, :, :Sk], ksc[:, :, :Sk], vc[:, :, :Sk // 32], vsc[:, :, :Sk // 32] = k, ks, v, vs
    kw = dict(causal=True, q_pos0=Sk - Sq, v_fmt=BLK)
    pd = mxfa.make_params(B, Hq, Hkv, Sq, Sk, D, **kw)
    ps = mxfa.make_params(B, Hq, Hkv, Sq, Sk, D, kv_stride=Lcap, **kw)
    for ws in (None, False):
        dense = mxfa.prefill(pd, q, qs, k, ks, v, vs, workspace=ws)
        strided = mxfa.prefill(ps, q, qs, kc, ksc, vc, vsc, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(strided, dense), ("workspace" if ws is None else "workspace-free", D)
    want = O.attention(oracle_params(_e3m2_params(pd)), np_(q), np_(qs), np_(k), np_(ks),
                       mxfa.e3m2_from_blk(np_(v)), np_(vs), block_n=mxfa.DEFAULT_BLOCK_N)
    rel, mab = errors(np_(strided), want)
    print(f"   strided BLK cache D={D}: rel-L2 {rel:.3e} max-abs {mab:.3e}", flush=True)
    assert rel <= REL_L2_TOL and mab <= MAX_ABS_TOL


def test_kv_append_blk_matches_one_shot_then_prefill():
    """Appends of ragged chunks keep the block-packed V cache equal to the oracle's one-shot
    E3M2 quantization of everything so far, packed (blocks past the open one untouched); a
    prefill over the finished cache equals the one over quantize_cols of the whole V."""
    B, H, L, D = 2, 3, 320, 128
    rng = np.random.default_rng(640)
    Kf = (rng.standard_normal((B, H, L, D)) * 2.0 ** rng.integers(-6, 6, (1, 1, L, 1))).astype(np.float32)
    Vf = (rng.standard_normal((B, H, L, D)) * 2.0 ** rng.integers(-6, 6, (1, 1, L, 1))).astype(np.float32)
    Vf[:, :, 40:44] = 0.0
    cache = mxfa.KvCache(B, H, D, L, v_fmt=BLK)
    assert tuple(cache.v.shape) == (B, H, L // 32, D, 24)
    sentinel = 0xA5
    cache.v.fill_(sentinel)
    cache.vs.fill_(sentinel)
    Kd, Vd = torch.from_numpy(Kf).to(DEV), torch.from_numpy(Vf).to(DEV)
    for n in [1, 5, 26, 32, 7, 33, 64, 1, 1, 30, 45, 75]:
        p0 = cache.length
        cache.append(Kd[:, :, p0:p0 + n].contiguous(), Vd[:, :, p0:p0 + n].contiguous())
        torch.cuda.synchronize()
        m = cache.length
        nb = -(-m // 32)
        Vp = np.zeros((B, H, nb * 32, D), np.float32)
        Vp[:, :, :m] = Vf[:, :, :m]
        vc, vs = O.quantize_cols(Vp, O.FMT_E3M2)
        np.testing.assert_array_equal(np_(cache.v)[:, :, :nb], mxfa.e3m2_to_blk(vc))
        np.testing.assert_array_equal(np_(cache.vs)[:, :, :nb], vs)
        if m < L:
            assert np.all(np_(cache.v)[:, :, nb:] == sentinel)
    Hq, Sq = 6, 64
    q, qs = mxfa.quantize_rows(torch.from_numpy(rng.standard_normal((B, Hq, Sq, D)).astype(np.float32)).to(DEV))
    v1, v1s = mxfa.quantize_cols(Vd, BLK)
    p = mxfa.make_params(B, Hq, H, Sq, L, D, causal=True, q_pos0=L - Sq, v_fmt=BLK)
    got = mxfa.prefill(p, q, qs, cache.k, cache.ks, cache.v, cache.vs)
    ref = mxfa.prefill(p, q, qs, cache.k, cache.ks, v1, v1s)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


@pytest.mark.parametrize("B,Hq,Hkv,L,D,softcap,p_rule,window", [
    (3, 8, 2, 480, 64, 0.0, mxfa.P_R1, 0),          # ragged last block (L % 64 = 32)
    (4, 32, 8, 1056, 128, 0.0, mxfa.P_R1, 0),       # ragged: the second 32-key block of the last is past L
    (2, 16, 8, 2080, 256, 30.0, mxfa.P_R1, 0),      # D = 256 kernel, softcap
    (2, 16, 4, 1024, 128, 50.0, mxfa.P_R2, 300),    # R2, window
    (1, 8, 8, 800, 256, 0.0, mxfa.P_R2, 0),
])
def test_decode_blk_matches_oracle_and_byte_e3m2(B, Hq, Hkv, L, D, softcap, p_rule, window):
    """Decode over block-packed E3M2 V: each 64-key block's 48 D bytes go unchanged into the
    wave's LDS slot (loads past seq_k / 32 blocks read 0); PV reads them as the fp6 operand.  Against the oracle (codes unpacked) and the byte-E3M2
    decode (same values: O within a few ulps)."""
    print(f"blk decode B{B} Hq{Hq} Hkv{Hkv} L{L} D{D} softcap {softcap} p_rule {p_rule} window {window}", flush=True)
    L32 = -(-L // 32) * 32
    fp, dev, host = gen_qkv(B, Hq, Hkv, 1, L32, D, 650 + D + L % 97, v_fmt=mxfa.FMT_E3M2)
    vb, vbs = mxfa.quantize_cols(fp["V"], BLK)
    kw = dict(causal=True, q_pos0=L - 1, softcap=softcap, p_rule=p_rule, window=window)
    p = mxfa.make_params(B, Hq, Hkv, 1, L32, D, v_fmt=BLK, **kw)
    pe = mxfa.make_params(B, Hq, Hkv, 1, L32, D, v_fmt=mxfa.FMT_E3M2, **kw)
    out = mxfa.decode(p, dev["q"], dev["qs"], dev["k"], dev["ks"], vb, vbs)
    ref = mxfa.decode(pe, dev["q"], dev["qs"], dev["k"], dev["ks"], dev["v"], dev["vs"])
    torch.cuda.synchronize()
    o = np_(out)
    assert np.all(np.isfinite(o))
    n_parts, _ = mxfa.decode_plan(p)
    want = O.attention(oracle_params(pe), host["q"], host["qs"], host["k"], host["ks"], host["v"], host["vs"],
                       block_n=mxfa.DEFAULT_BLOCK_N, n_parts=n_parts)
    rel, mab = errors(o, want)
    drel, dmab = errors(o, np_(ref))
    print(f"   n_parts {n_parts}: rel-L2 {rel:.3e} max-abs {mab:.3e}; vs byte E3M2 rel-L2 {drel:.2e} max-abs "
          f"{dmab:.2e} (bit-identical: {torch.equal(out, ref)})", flush=True)
    assert rel <= REL_L2_TOL and mab <= MAX_ABS_TOL
    assert drel <= 1e-5 and dmab <= 1e-4


def test_decode_blk_over_appended_cache_and_noalloc():
    """The serving loop on a block-packed cache: prefill-sized append, then one-token appends
    with a decode after each (seq_k = length rounded up to 32, kv_stride = max_len); each
    decode against the oracle on the unpacked cache, and mxfa_decode_noalloc equal to
    mxfa_decode bit for bit."""
    B, Hq, H, L, D = 2, 8, 2, 256, 128
    rng = np.random.default_rng(660)
    Kf = rng.standard_normal((B, H, L, D)).astype(np.float32)
    Vf = rng.standard_normal((B, H, L, D)).astype(np.float32)
    Qf = rng.standard_normal((3, B, Hq, 1, D)).astype(np.float32)
    cache = mxfa.KvCache(B, H, D, L, v_fmt=BLK)
    Kd, Vd = torch.from_numpy(Kf).to(DEV), torch.from_numpy(Vf).to(DEV)
    mxfa.init()
    for step, n in enumerate([161, 1, 1]):
        p0 = cache.length
        cache.append(Kd[:, :, p0:p0 + n].contiguous(), Vd[:, :, p0:p0 + n].contiguous())
        q, qs = mxfa.quantize_rows(torch.from_numpy(Qf[step]).to(DEV))
        p = cache.decode_params(Hq)
        out = mxfa.decode(p, q, qs, cache.k, cache.ks, cache.v, cache.vs)
        out_na = torch.empty_like(out)
        mxfa.decode_noalloc(p, q, qs, cache.k, cache.ks, cache.v, cache.vs, out_na)
        torch.cuda.synchronize()
        assert torch.equal(out, out_na)
        sk = p.seq_k
        pe = mxfa.make_params(B, Hq, H, 1, sk, D, causal=True, q_pos0=cache.length - 1, v_fmt=mxfa.FMT_E3M2)
        n_parts, _ = mxfa.decode_plan(pe)
        v_bytes = mxfa.e3m2_from_blk(np_(cache.v)[:, :, :sk // 32])
        c = np.ascontiguousarray
        want = O.attention(oracle_params(pe), np_(q), np_(qs), c(np_(cache.k)[:, :, :sk]), c(np_(cache.ks)[:, :, :sk]),
                           v_bytes, c(np_(cache.vs)[:, :, :sk // 32]), block_n=mxfa.DEFAULT_BLOCK_N, n_parts=n_parts)
        rel, mab = errors(np_(out), want)
        print(f"   length {cache.length}: rel-L2 {rel:.3e} max-abs {mab:.3e}", flush=True)
        assert rel <= REL_L2_TOL and mab <= MAX_ABS_TOL


def test_trace_refuses_blk():
    """The stage trace reads V as codes one per byte: block-packed V is refused with
    MXFA_ERR_UNSUPPORTED before anything is launched."""
    B, Hq, Hkv, Sk, D = 1, 2, 1, 64, 64
    z = lambda *s: torch.zeros(s, dtype=torch.uint8, device=DEV)  # noqa: E731
    k, ks = z(B, Hkv, Sk, D), z(B, Hkv, Sk, D // 32)
    v, vs = z(B, Hkv, Sk // 32, D, 24), z(B, Hkv, Sk // 32, D)
    pp = mxfa.make_params(B, Hq, Hkv, 32, Sk, D, v_fmt=BLK)
    with pytest.raises(mxfa.MxfaError) as e:
        mxfa.prefill_trace(pp, z(B, Hq, 32, D), z(B, Hq, 32, D // 32), k, ks, v, vs, 0, 0)
    assert e.value.status == 2
