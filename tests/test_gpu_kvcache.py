"""GPU parity of the KV-cache append (mxfa_kv_append): after every append of a ragged
sequence of chunks, the cache equals the oracle's one-shot R1 quantization of everything
appended so far (K rows; V in 32-token blocks, zero-padded) bit for bit, and decode over
the appended cache matches the oracle."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import mxfa  # noqa: E402
import oracle as O  # noqa: E402
from gpuhelp import DEV, MAX_ABS_TOL, REL_L2_TOL, errors, np_, oracle_params, sweep_seeds  # noqa: E402

pytestmark = pytest.mark.gpu


def expected_cache(Kf, Vf, n, fmt):
    """Oracle: K rows [.., :n, :] and V blocks of the zero-padded first n tokens."""
    B, H, _, D = Kf.shape
    n32 = -(-n // 32) * 32
    kc, ks = O.quantize_rows(np.ascontiguousarray(Kf[:, :, :n]).reshape(-1, D), O.FMT_E4M3)
    Vp = np.zeros((B, H, n32, D), np.float32)
    Vp[:, :, :n] = Vf[:, :, :n]
    vc, vs = O.quantize_cols(Vp, fmt)
    return kc.reshape(B, H, n, D), ks.reshape(B, H, n, D // 32), vc, vs


@pytest.mark.parametrize("D,fmt", [(128, mxfa.FMT_E4M3), (64, mxfa.FMT_E3M2), (256, mxfa.FMT_E4M3)])
def test_append_matches_one_shot_quantization(D, fmt):
    B, H, L = 2, 3, 320
    rng = np.random.default_rng(400 + D)
    Kf = (rng.standard_normal((B, H, L, D)) * 2.0 ** rng.integers(-6, 6, (1, 1, L, 1))).astype(np.float32)
    Vf = (rng.standard_normal((B, H, L, D)) * 2.0 ** rng.integers(-6, 6, (1, 1, L, 1))).astype(np.float32)
    Vf[:, :, 40:44] = 0.0                                            # all-zero rows inside a block
    cache = mxfa.KvCache(B, H, D, L, v_fmt=fmt)
    sentinel = 0xA5
    for t in (cache.k, cache.ks, cache.v, cache.vs):
        t.fill_(sentinel)
    chunks = [1, 5, 26, 32, 7, 33, 64, 1, 1, 30, 45, 75]             # 320 tokens: starts mid-block, spans blocks
    assert sum(chunks) == L
    Kd, Vd = torch.from_numpy(Kf).to(DEV), torch.from_numpy(Vf).to(DEV)
    for n in chunks:
        p0 = cache.length
        cache.append(Kd[:, :, p0:p0 + n].contiguous(), Vd[:, :, p0:p0 + n].contiguous())
        torch.cuda.synchronize()
        m = cache.length
        m32 = -(-m // 32) * 32
        kc, ks, vc, vs = expected_cache(Kf, Vf, m, fmt)
        np.testing.assert_array_equal(np_(cache.k)[:, :, :m], kc)
        np.testing.assert_array_equal(np_(cache.ks)[:, :, :m], ks)
        np.testing.assert_array_equal(np_(cache.v)[:, :, :m32], vc)
        np.testing.assert_array_equal(np_(cache.vs)[:, :, :m32 // 32], vs)
        if m < L:                                                     # nothing past the block is written
            assert np.all(np_(cache.k)[:, :, m:] == sentinel)
            assert np.all(np_(cache.v)[:, :, m32:] == sentinel)


@pytest.mark.parametrize("i", sweep_seeds(range(6), "MXFA_KV_SEEDS"))
def test_append_sweep(i):
    """Seeded random append sequences (chunks of 1-100 tokens, the cache filled to a random
    length) for D 64/128/256 and V as E4M3, E3M2 bytes or block-packed E3M2: after every
    append the cache equals the oracle's one-shot quantization of everything so far, and
    nothing past the open block is written.  MXFA_KV_SEEDS=0-200 runs it longer."""
    rng = np.random.default_rng(52000 + i)
    D = int(rng.choice([64, 128, 256]))
    fmt = (mxfa.FMT_E4M3, mxfa.FMT_E3M2, mxfa.FMT_E3M2_BLK)[i % 3]
    B, H = int(rng.integers(1, 3)), int(rng.integers(1, 4))
    L = 32 * int(rng.integers(2, 24))
    Kf = (rng.standard_normal((B, H, L, D)) * 2.0 ** rng.integers(-8, 8, (1, 1, L, 1))).astype(np.float32)
    Vf = (rng.standard_normal((B, H, L, D)) * 2.0 ** rng.integers(-8, 8, (1, 1, L, 1))).astype(np.float32)
    cache = mxfa.KvCache(B, H, D, L, v_fmt=fmt)
    sentinel = 0x5A
    for t_ in (cache.k, cache.ks, cache.v, cache.vs):
        t_.fill_(sentinel)
    Kd, Vd = torch.from_numpy(Kf).to(DEV), torch.from_numpy(Vf).to(DEV)
    target = int(rng.integers(1, L + 1))
    print(f"append sweep {i}: B{B} H{H} D{D} L{L} fmt {fmt} to {target}", flush=True)
    while cache.length < target:
        p0 = cache.length
        n = min(int(rng.integers(1, 101)), target - p0)
        cache.append(Kd[:, :, p0:p0 + n].contiguous(), Vd[:, :, p0:p0 + n].contiguous())
        torch.cuda.synchronize()
        m = cache.length
        nb = -(-m // 32)
        kc, ks, vc, vs = expected_cache(Kf, Vf, m, mxfa.FMT_E4M3 if fmt == mxfa.FMT_E4M3 else mxfa.FMT_E3M2)
        np.testing.assert_array_equal(np_(cache.k)[:, :, :m], kc)
        np.testing.assert_array_equal(np_(cache.ks)[:, :, :m], ks)
        if fmt == mxfa.FMT_E3M2_BLK:
            np.testing.assert_array_equal(np_(cache.v)[:, :, :nb], mxfa.e3m2_to_blk(vc))
            assert np.all(np_(cache.v)[:, :, nb:] == sentinel)
        else:
            np.testing.assert_array_equal(np_(cache.v)[:, :, :32 * nb], vc)
            assert np.all(np_(cache.v)[:, :, 32 * nb:] == sentinel)
        np.testing.assert_array_equal(np_(cache.vs)[:, :, :nb], vs)
        assert np.all(np_(cache.k)[:, :, m:] == sentinel)


def test_decode_over_appended_cache():
    """Decode at a length that is not a multiple of 32 (seq_k rounded up, q_pos0 = L - 1
    masks the padding), cache built by appends, against the oracle on that cache."""
    B, Hq, Hkv, D, Lcap = 4, 8, 2, 128, 512
    n = 389
    rng = np.random.default_rng(410)
    Kf = rng.standard_normal((B, Hkv, Lcap, D)).astype(np.float32)
    Vf = rng.standard_normal((B, Hkv, Lcap, D)).astype(np.float32)
    cache = mxfa.KvCache(B, Hkv, D, Lcap)
    Kd, Vd = torch.from_numpy(Kf).to(DEV), torch.from_numpy(Vf).to(DEV)
    for c in (100, 1, 131, 157):
        p0 = cache.length
        cache.append(Kd[:, :, p0:p0 + c].contiguous(), Vd[:, :, p0:p0 + c].contiguous())
    assert cache.length == n
    Q = torch.empty((B, Hq, 1, D), dtype=torch.float32, device=DEV)
    mxfa.fill_normal(Q, 411)
    q, qs = mxfa.quantize_rows(Q)
    sk = -(-n // 32) * 32
    p = mxfa.make_params(B, Hq, Hkv, 1, sk, D, causal=True, q_pos0=n - 1)
    k, ks = cache.k[:, :, :sk].contiguous(), cache.ks[:, :, :sk].contiguous()
    v, vs = cache.v[:, :, :sk].contiguous(), cache.vs[:, :, :sk // 32].contiguous()
    o = mxfa.decode(p, q, qs, k, ks, v, vs)
    torch.cuda.synchronize()
    n_parts, _ = mxfa.decode_plan(p)
    want = O.attention(oracle_params(p), np_(q), np_(qs), np_(k), np_(ks), np_(v), np_(vs),
                       block_n=mxfa.DEFAULT_BLOCK_N, n_parts=n_parts)
    rel, mab = errors(np_(o), want)
    print(f"   decode over appended cache: rel-L2 {rel:.3e} max-abs {mab:.3e}", flush=True)
    assert rel <= REL_L2_TOL and mab <= MAX_ABS_TOL


def test_decode_in_place_on_cache_with_capacity():
    """Decode reads the cache tensors in place (kv_stride = max_len > seq_k) for several
    (batch, KV head) pairs: the same O, bit for bit, as decoding contiguous copies of the
    first seq_k keys, and within tolerance of the oracle."""
    B, Hq, Hkv, D, Lcap, n = 3, 16, 4, 128, 1024, 333
    rng = np.random.default_rng(420)
    cache = mxfa.KvCache(B, Hkv, D, Lcap)
    Kd = torch.from_numpy(rng.standard_normal((B, Hkv, n, D)).astype(np.float32)).to(DEV)
    Vd = torch.from_numpy(rng.standard_normal((B, Hkv, n, D)).astype(np.float32)).to(DEV)
    cache.append(Kd[:, :, :200].contiguous(), Vd[:, :, :200].contiguous())
    cache.append(Kd[:, :, 200:].contiguous(), Vd[:, :, 200:].contiguous())
    Q = torch.empty((B, Hq, 1, D), dtype=torch.float32, device=DEV)
    mxfa.fill_normal(Q, 421)
    q, qs = mxfa.quantize_rows(Q)
    p = cache.decode_params(Hq)
    assert p.kv_stride == Lcap and p.seq_k == 352 and p.q_pos0 == n - 1
    got = mxfa.decode(p, q, qs, cache.k, cache.ks, cache.v, cache.vs)
    sk = p.seq_k
    k, ks = cache.k[:, :, :sk].contiguous(), cache.ks[:, :, :sk].contiguous()
    v, vs = cache.v[:, :, :sk].contiguous(), cache.vs[:, :, :sk // 32].contiguous()
    pc = mxfa.make_params(B, Hq, Hkv, 1, sk, D, causal=True, q_pos0=n - 1)
    dense = mxfa.decode(pc, q, qs, k, ks, v, vs)
    # prefill over the cache in place (one query row per head at the last position)
    pp = mxfa.make_params(B, Hq, Hkv, 1, sk, D, causal=True, q_pos0=n - 1, kv_stride=Lcap)
    pre_inplace = mxfa.prefill(pp, q, qs, cache.k, cache.ks, cache.v, cache.vs)
    pre_dense = mxfa.prefill(pc, q, qs, k, ks, v, vs)
    torch.cuda.synchronize()
    assert torch.equal(got, dense)
    assert torch.equal(pre_inplace, pre_dense)
    n_parts, _ = mxfa.decode_plan(pc)
    want = O.attention(oracle_params(pc), np_(q), np_(qs), np_(k), np_(ks), np_(v), np_(vs),
                       block_n=mxfa.DEFAULT_BLOCK_N, n_parts=n_parts)
    rel, mab = errors(np_(got), want)
    print(f"   in-place decode: rel-L2 {rel:.3e} max-abs {mab:.3e}", flush=True)
    assert rel <= REL_L2_TOL and mab <= MAX_ABS_TOL


@pytest.mark.parametrize("D,fmt", [(64, mxfa.FMT_E3M2), (128, mxfa.FMT_E4M3), (256, mxfa.FMT_E3M2),
                                   (256, mxfa.FMT_E4M3)])
def test_prefill_in_place_on_strided_cache(D, fmt):
    """Prefill with several query tiles (Sq > 32) over caches whose rows are kv_stride >
    seq_k apart, the rows past seq_k holding garbage codes: the workspace prefill (its
    pre-pass reads K -- and E3M2 V -- at the cache stride) and the workspace-free kernel
    (K codes and scales read at the cache stride, widened in LDS) give O bit for bit equal
    to the same calls on dense copies of the first seq_k keys, within tolerance of the oracle."""
    B, Hq, Hkv, Sq, Sk, Lcap = 2, 4, 2, 96, 160, 256
    rng = np.random.default_rng(430 + D + 7 * fmt)
    Q = torch.from_numpy(rng.standard_normal((B, Hq, Sq, D)).astype(np.float32)).to(DEV)
    K = torch.from_numpy(rng.standard_normal((B, Hkv, Sk, D)).astype(np.float32)).to(DEV)
    V = torch.from_numpy(rng.standard_normal((B, Hkv, Sk, D)).astype(np.float32)).to(DEV)
    q, qs = mxfa.quantize_rows(Q)
    k, ks = mxfa.quantize_rows(K)
    v, vs = mxfa.quantize_cols(V, fmt)
    garbage = lambda shape: torch.from_numpy(rng.integers(0, 256, shape, dtype=np.uint8)).to(DEV)  # noqa: E731
    kc, ksc = garbage((B, Hkv, Lcap, D)), garbage((B, Hkv, Lcap, D // 32))
    vc, vsc = garbage((B, Hkv, Lcap, D)), garbage((B, Hkv, Lcap // 32, D))
    kc[:, :, :Sk], ksc[:, :, :Sk], vc[:, :, :Sk], vsc[:, :, :Sk // 32] = k, ks, v, vs
    kw = dict(causal=True, q_pos0=Sk - Sq, v_fmt=fmt)
    pd = mxfa.make_params(B, Hq, Hkv, Sq, Sk, D, **kw)
    ps = mxfa.make_params(B, Hq, Hkv, Sq, Sk, D, kv_stride=Lcap, **kw)
    for ws in (None, False):
        dense = mxfa.prefill(pd, q, qs, k, ks, v, vs, workspace=ws)
        strided = mxfa.prefill(ps, q, qs, kc, ksc, vc, vsc, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(strided, dense), ("workspace" if ws is None else "workspace-free", D, fmt)
    want = O.attention(oracle_params(pd), np_(q), np_(qs), np_(k), np_(ks), np_(v), np_(vs),
                       block_n=mxfa.DEFAULT_BLOCK_N)
    rel, mab = errors(np_(strided), want)
    print(f"   strided-cache prefill D={D} fmt={fmt}: rel-L2 {rel:.3e} max-abs {mab:.3e}", flush=True)
    assert rel <= REL_L2_TOL and mab <= MAX_ABS_TOL
