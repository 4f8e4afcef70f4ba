"""GPU parity of MXFP8 prefill and decode against the oracle (same block size and
split schedule), to the north_star tolerance: rel-L2 <= 5e-3 and max-abs <= 2e-2.
Operands are generated and quantized on the GPU; the oracle first re-quantizes the
same fp32 values and must reproduce the codes bit for bit."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import mxfa  # noqa: E402
import oracle as O  # noqa: E402
from gpuhelp import DEV, MAX_ABS_TOL, REL_L2_TOL, errors, explain_max_abs, gen_qkv, np_, oracle_params  # noqa: E402

pytestmark = pytest.mark.gpu


def run_case(B, Hq, Hkv, Sq, Sk, D, causal=False, q_pos0=0, window=0, softcap=0.0, v_fmt=mxfa.FMT_E4M3,
             seed=0, outlier_p=0.0, q_mul=1.0, heads=None, check_codes=True, p_rule=mxfa.P_R1, max_rows=8):
    print(f"case B{B} Hq{Hq} Hkv{Hkv} Sq{Sq} Sk{Sk} D{D} causal{causal} q_pos0 {q_pos0} window {window} "
          f"softcap {softcap} v_fmt {v_fmt} seed {seed} p_rule {p_rule}", flush=True)
    fp, dev, host = gen_qkv(B, Hq, Hkv, Sq, Sk, D, seed, outlier_p=outlier_p, q_mul=q_mul, v_fmt=v_fmt)
    if check_codes:
        oq, oqs = O.quantize_rows(np_(fp["Q"]), O.FMT_E4M3)
        np.testing.assert_array_equal(host["q"], oq)
        np.testing.assert_array_equal(host["qs"], oqs)
        ov, ovs = O.quantize_cols(np_(fp["V"]), v_fmt)
        np.testing.assert_array_equal(host["v"], ov)
        np.testing.assert_array_equal(host["vs"], ovs)
    p = mxfa.make_params(B, Hq, Hkv, Sq, Sk, D, causal=causal, q_pos0=q_pos0, window=window, softcap=softcap,
                         v_fmt=v_fmt, p_rule=p_rule)
    out = torch.full((B, Hq, Sq, D), float("nan"), dtype=torch.float32, device=DEV)
    mxfa.prefill(p, dev["q"], dev["qs"], dev["k"], dev["ks"], dev["v"], dev["vs"], out=out)
    # the workspace-free kernel (mxfa_prefill: K widened to bf16 in LDS): with E4M3 V the same
    # arithmetic in the same order as the workspace kernel (bit-identical O); with E3M2 V the
    # PV MFMA reads V as E5M2 (O within a few ulps of the workspace kernel's), checked against
    # the oracle
    out_nw = torch.full_like(out, float("nan"))
    mxfa.prefill(p, dev["q"], dev["qs"], dev["k"], dev["ks"], dev["v"], dev["vs"], out=out_nw, workspace=False)
    torch.cuda.synchronize()
    same_kernel_order = v_fmt == mxfa.FMT_E4M3
    if same_kernel_order:
        assert torch.equal(out, out_nw), "mxfa_prefill_ws and mxfa_prefill differ"
    o = np_(out)
    assert np.all(np.isfinite(o)), "coverage: some O elements were not written"
    want = O.attention(oracle_params(p), host["q"], host["qs"], host["k"], host["ks"], host["v"], host["vs"],
                       block_n=mxfa.DEFAULT_BLOCK_N, heads=heads)
    if heads is not None:
        idx = np.array(heads)
        o = o.reshape(B * Hq, Sq, D)[idx]
        want = want.reshape(B * Hq, Sq, D)[idx]
    rel, mab = errors(o, want)
    print(f"   rel-L2 {rel:.3e} max-abs {mab:.3e}", flush=True)
    assert rel <= REL_L2_TOL
    if mab > MAX_ABS_TOL:
        # only where P code boundaries hit between fp32 and double P account for every excess
        assert heads is None, "max-abs bound exceeded"
        explain_max_abs(p, dev, host, o, want, max_rows=max_rows)
    if not same_kernel_order:
        o2 = np_(out_nw)
        assert np.all(np.isfinite(o2))
        if heads is not None:
            o2 = o2.reshape(B * Hq, Sq, D)[idx]
        rel2, mab2 = errors(o2, want)
        print(f"   workspace-free kernel: rel-L2 {rel2:.3e} max-abs {mab2:.3e}", flush=True)
        assert rel2 <= REL_L2_TOL
        if mab2 > MAX_ABS_TOL:
            assert heads is None, "max-abs bound exceeded"
            explain_max_abs(p, dev, host, o2, want, max_rows=max_rows)
    return p, dev, out


def test_config1_single_head_noncausal():
    """B=1 H=1 S=256 D=64, non-causal."""
    run_case(1, 1, 1, 256, 256, 64, seed=1)


def test_reference_gqa_tile():
    """The reference GQA kernel's own case: NQ=8, NKV=2, Sq=64, Sk=256, d=64, q_pos0=64
    (kernels/regen_data.sh:31-34)."""
    run_case(1, 8, 2, 64, 256, 64, causal=True, q_pos0=64, seed=2)


@pytest.mark.parametrize("D", [64, 128, 256])
def test_causal_gqa_head_dims(D):
    run_case(2, 8, 2, 160, 160, D, causal=True, seed=3 + D)


def test_ragged_lengths():
    """Sq not a multiple of the 32-row wave tile; Sk not a multiple of the 64-key block."""
    run_case(1, 4, 4, 77, 96, 128, causal=False, seed=5)
    run_case(2, 4, 1, 45, 224, 128, causal=True, q_pos0=179, seed=6)


def test_gemma_softcap_window_e3m2():
    """Reference gemma variant semantics: softcap before max, sliding window, V in E3M2."""
    run_case(1, 4, 2, 384, 384, 256, causal=True, window=128, softcap=50.0, v_fmt=mxfa.FMT_E3M2, seed=7)


def test_softcap_saturated_queries():
    """The reference's softcap stress: queries x50 so the cap saturates."""
    run_case(1, 2, 1, 128, 128, 128, causal=True, softcap=50.0, q_mul=50.0, seed=8)


def test_softcap_saturation_scale_ties():
    """Softcap 30 with 1% x20 outliers over long non-causal rows with a window: many scores
    saturate to within fp32 precision of the cap, so a tile maximum that is ~1e-7 below the
    row maximum in double equals it in fp32, and the tile's P scale lands on the other side of
    R1's power-of-two boundary (the block's largest P requantizes to 256 * 2^-8 = 1 instead of
    448 * 2^-9 = 0.875).  Every element past max-abs (318 in 87 rows here) must be traced to
    such a scale tie, a code tie or R1's flush boundary (found by an exploratory sweep)."""
    run_case(1, 32, 4, 838, 4992, 64, window=257, softcap=30.0, outlier_p=0.01, seed=77033, max_rows=200)


def test_outliers():
    """1% of elements x20, as in the S=4096 GQA headline config."""
    run_case(1, 8, 2, 256, 256, 128, causal=True, outlier_p=0.01, seed=9)


def test_fully_masked_rows_are_zero():
    B, H, Sq, Sk, D = 1, 2, 32, 64, 64
    p, dev, out = run_case(B, H, H, Sq, Sk, D, causal=True, q_pos0=200, window=100, seed=10)
    assert np.all(np_(out) == 0.0)


def test_deterministic():
    p, dev, out = run_case(1, 4, 2, 256, 256, 128, causal=True, seed=11)
    out2 = mxfa.prefill(p, dev["q"], dev["qs"], dev["k"], dev["ks"], dev["v"], dev["vs"])
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


@pytest.mark.parametrize("cfg", ["c2", "c3", "c4"])
def test_baseline_configs_all_heads(cfg):
    """Full BASELINE shapes, every head against the oracle (the threaded C oracle takes a
    few seconds per configuration)."""
    if cfg == "c2":
        run_case(4, 16, 16, 2048, 2048, 128, causal=True, seed=21, check_codes=False)
    elif cfg == "c3":
        run_case(2, 32, 8, 4096, 4096, 128, causal=True, outlier_p=0.01, seed=22, check_codes=False)
    else:
        run_case(1, 16, 8, 8192, 8192, 256, causal=True, window=4096, softcap=50.0, v_fmt=mxfa.FMT_E3M2, seed=23,
                 check_codes=False)


def test_softcap_stress_config4_shape():
    """The reference's softcap stress (Q x 50, kernels/flash_attention_mx_gemma/fa_gen_data.py:
    77-79,98) at the Gemma config's full shape: B=1 Hq=16 Hkv=8 S=8192 D=256, window 4096,
    softcap 50, E3M2 V; every head against the oracle."""
    run_case(1, 16, 8, 8192, 8192, 256, causal=True, window=4096, softcap=50.0, v_fmt=mxfa.FMT_E3M2, seed=24,
             q_mul=50.0, check_codes=False)


def run_decode(B, Hq, Hkv, L, D, seed, heads=None, v_fmt=mxfa.FMT_E4M3, softcap=0.0, p_rule=mxfa.P_R1):
    print(f"decode B{B} Hq{Hq} Hkv{Hkv} L{L} D{D} seed {seed} p_rule {p_rule}", flush=True)
    fp, dev, host = gen_qkv(B, Hq, Hkv, 1, L, D, seed, v_fmt=v_fmt)
    p = mxfa.make_params(B, Hq, Hkv, 1, L, D, causal=True, q_pos0=L - 1, softcap=softcap, v_fmt=v_fmt,
                         p_rule=p_rule)
    n_parts, _ = mxfa.decode_plan(p)
    out = torch.full((B, Hq, 1, D), float("nan"), dtype=torch.float32, device=DEV)
    mxfa.decode(p, dev["q"], dev["qs"], dev["k"], dev["ks"], dev["v"], dev["vs"], out=out)
    torch.cuda.synchronize()
    o = np_(out)
    assert np.all(np.isfinite(o))
    want = O.attention(oracle_params(p), host["q"], host["qs"], host["k"], host["ks"], host["v"], host["vs"],
                       block_n=mxfa.DEFAULT_BLOCK_N, n_parts=n_parts, heads=heads)
    if heads is not None:
        idx = np.array(heads)
        o = o.reshape(B * Hq, D)[idx]
        want = want.reshape(B * Hq, D)[idx]
    rel, mab = errors(o, want)
    print(f"   n_parts {n_parts} rel-L2 {rel:.3e} max-abs {mab:.3e}", flush=True)
    assert rel <= REL_L2_TOL and mab <= MAX_ABS_TOL
    return p, dev, out


def test_decode_small():
    run_decode(4, 32, 8, 1024, 128, seed=30)


def test_decode_group_32():
    """32 query heads per KV head, the largest group decode takes: all 32 score columns
    are valid and the partials merge in the combine kernel."""
    run_decode(2, 32, 1, 1024, 128, seed=34)
    run_decode(1, 64, 2, 640, 64, seed=35)


def test_decode_ragged_and_e3m2():
    run_decode(3, 8, 2, 480, 64, seed=31, v_fmt=mxfa.FMT_E3M2)
    run_decode(2, 16, 8, 2080, 256, seed=32, softcap=30.0)


def test_long_context_decode_and_prefill():
    """Long caches: decode over 262,144 keys (hundreds of key blocks per partial, the split
    plan at its widest), and a 64-query chunk prefilled at the end of a 131,072-key cache (few
    work items, 2,048 key blocks each) at D = 256 with softcap and E3M2 V."""
    run_decode(1, 8, 1, 262144, 128, seed=36)
    run_case(1, 4, 2, 64, 131072, 256, causal=True, q_pos0=131072 - 64, softcap=30.0, v_fmt=mxfa.FMT_E3M2,
             seed=37, check_codes=False)


def test_gqa_groups_not_powers_of_two():
    """Query heads per KV head of 3, 6, 7 and 24: the workgroup's heads-per-wave split falls
    back to the largest power of two dividing the group (1, 2, 1, 8)."""
    run_case(1, 9, 3, 96, 160, 128, causal=True, q_pos0=64, seed=38)
    run_case(2, 12, 2, 70, 96, 64, softcap=30.0, seed=39, v_fmt=mxfa.FMT_E3M2)
    run_case(1, 7, 1, 130, 256, 256, causal=True, q_pos0=126, window=100, seed=40)
    run_decode(2, 24, 1, 800, 128, seed=41)
    run_decode(3, 21, 3, 480, 64, seed=42, v_fmt=mxfa.FMT_E3M2)


def test_decode_config5_all_heads():
    """B=64, Hq=32, Hkv=8, D=128, KV length 8192."""
    p, dev, out = run_decode(64, 32, 8, 8192, 128, seed=33)
    out2 = mxfa.decode(p, dev["q"], dev["qs"], dev["k"], dev["ks"], dev["v"], dev["vs"])
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


def test_decode_d256_full_shape():
    """Decode at D = 256 over 32 caches of 8,192 tokens (Gemma heads: Hq 16, Hkv 8, softcap
    50; the shape bench.py times), every head against the oracle; a second call gives the
    same O bit for bit."""
    p, dev, out = run_decode(32, 16, 8, 8192, 256, seed=37, softcap=50.0)
    out2 = mxfa.decode(p, dev["q"], dev["qs"], dev["k"], dev["ks"], dev["v"], dev["vs"])
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


@pytest.mark.parametrize("B,Hq,Hkv,L,D,waves,window,softcap", [
    (4, 32, 8, 1024, 128, 32, 0, 0.0),        # 1 partial per head
    (4, 32, 8, 1024, 128, 64, 0, 0.0),        # 2 partials
    (4, 32, 8, 1024, 128, 128, 300, 0.0),     # 4 partials, window (partials start past block 0)
    (3, 8, 2, 480, 64, 18, 0, 30.0),          # 3 -> 4 partials, ragged last block, softcap, D = 64
    (2, 64, 4, 1056, 128, 16, 0, 0.0),        # group 16, ragged last block
    (4, 32, 8, 1024, 128, 256, 0, 0.0),       # 8 partials: not fused, both runs use the kernel
    (2, 16, 8, 1024, 256, 32, 0, 50.0),       # D = 256 (one workgroup per CU): 2 partials, softcap
    (2, 16, 8, 1056, 256, 64, 200, 0.0),      # D = 256: 4 partials, window, ragged last block
    (1, 32, 2, 512, 256, 4, 0, 0.0),          # D = 256, group 16: merge slots full
    (2, 16, 4, 2048, 256, 128, 0, 0.0),       # D = 256: 16 partials through the kernel
])
def test_decode_fused_merge_matches_combine_kernel(monkeypatch, B, Hq, Hkv, L, D, waves, window, softcap):
    """The in-workgroup merge of the interleaved partials (one launch) and
    mxfa_decode_combine (two launches) give bit-identical O: same partials, same formula,
    same order."""
    print(f"decode fused-vs-kernel B{B} Hq{Hq} Hkv{Hkv} L{L} D{D} waves {waves}", flush=True)
    monkeypatch.setenv("MXFA_DECODE_WAVES", str(waves))
    fp, dev, host = gen_qkv(B, Hq, Hkv, 1, L, D, seed=40 + waves)
    p = mxfa.make_params(B, Hq, Hkv, 1, L, D, causal=True, q_pos0=L - 1, window=window, softcap=softcap)
    args = (p, dev["q"], dev["qs"], dev["k"], dev["ks"], dev["v"], dev["vs"])
    fused = mxfa.decode(*args)
    monkeypatch.setenv("MXFA_DECODE_COMBINE", "kernel")
    combined = mxfa.decode(*args)
    torch.cuda.synchronize()
    assert torch.isfinite(fused).all()
    assert torch.equal(fused, combined)
    n_parts, _ = mxfa.decode_plan(p)
    want = O.attention(oracle_params(p), host["q"], host["qs"], host["k"], host["ks"], host["v"], host["vs"],
                       block_n=mxfa.DEFAULT_BLOCK_N, n_parts=n_parts)
    rel, mab = errors(np_(fused), want)
    assert rel <= REL_L2_TOL and mab <= MAX_ABS_TOL


# ---- P rule R2: the reference device kernels' truncating "target-0" requant of bf16 P
# (kernels/flash_attention_mx_gqa/flash_mx_impl.hpp:53-77, 366-388), same tolerance
# against the oracle run with the same rule.

def test_r2_reference_gqa_tile():
    p, dev, out = run_case(1, 8, 2, 64, 256, 64, causal=True, q_pos0=64, seed=2, p_rule=mxfa.P_R2)
    p1 = mxfa.make_params(1, 8, 2, 64, 256, 64, causal=True, q_pos0=64)
    out1 = mxfa.prefill(p1, dev["q"], dev["qs"], dev["k"], dev["ks"], dev["v"], dev["vs"])
    torch.cuda.synchronize()
    assert not torch.equal(out, out1)                 # the rule is in effect


@pytest.mark.parametrize("D", [64, 128, 256])
def test_r2_causal_gqa_head_dims(D):
    run_case(2, 8, 2, 160, 160, D, causal=True, seed=40 + D, p_rule=mxfa.P_R2)


def test_r2_ragged_softcap_window_e3m2():
    run_case(2, 4, 1, 45, 224, 128, causal=True, q_pos0=179, seed=41, p_rule=mxfa.P_R2)
    run_case(1, 4, 2, 384, 384, 256, causal=True, window=128, softcap=50.0, v_fmt=mxfa.FMT_E3M2, seed=42,
             p_rule=mxfa.P_R2)
    run_case(1, 8, 2, 256, 256, 128, causal=True, outlier_p=0.01, seed=43, p_rule=mxfa.P_R2)


def test_r2_config3_all_heads():
    run_case(2, 32, 8, 4096, 4096, 128, causal=True, outlier_p=0.01, seed=44, check_codes=False,
             p_rule=mxfa.P_R2)


def test_r2_decode():
    run_decode(4, 32, 8, 1024, 128, seed=45, p_rule=mxfa.P_R2)
    run_decode(3, 8, 2, 480, 64, seed=46, v_fmt=mxfa.FMT_E3M2, p_rule=mxfa.P_R2)
    run_decode(2, 16, 8, 2080, 256, seed=47, softcap=30.0, p_rule=mxfa.P_R2)


def test_reference_format_operands():
    """Operands exported to the reference's fa_data.h layout (header text) and imported
    back give the same prefill output bit for bit (the omitted key blocks are causally
    masked), under both P rules."""
    import fa_data as F
    Hq, Hkv, Sq, Sk, D, q_pos0 = 8, 2, 64, 256, 64, 64
    fp, dev, host = gen_qkv(1, Hq, Hkv, Sq, Sk, D, 50)
    names = ("q", "qs", "k", "ks", "v", "vs")
    fd = F.read_header(F.header_text(F.export_fa_data(*(host[n] for n in names), block_n=64, q_pos0=q_pos0)))
    imp, prm = F.import_fa_data(fd)
    assert prm["block_n"] == mxfa.DEFAULT_BLOCK_N
    idev = [torch.from_numpy(a).to(DEV) for a in imp]
    for rule in (mxfa.P_R1, mxfa.P_R2):
        p = mxfa.make_params(1, prm["Hq"], prm["Hkv"], prm["Sq"], prm["Sk"], prm["D"], causal=prm["causal"],
                             q_pos0=prm["q_pos0"], scale=prm["scale"], p_rule=rule)
        want = mxfa.prefill(p, *(dev[n] for n in names))
        got = mxfa.prefill(p, *idev)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
