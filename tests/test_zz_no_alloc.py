"""mxfa_decode_noalloc (the decode entry point that allocates nothing: its partials live in
the library's per-device scratch array) against mxfa_decode with a caller workspace: the
same O bit for bit, on consecutive calls whose second input is smaller, on the paths that
use the scratch (partials merged by the combine kernel: group 32, D = 256) and on the
in-workgroup merge path."""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import mxfa  # noqa: E402
import oracle as O  # noqa: E402
from gpuhelp import DEV, MAX_ABS_TOL, REL_L2_TOL, errors, gen_qkv, np_, oracle_params  # noqa: E402

pytestmark = pytest.mark.gpu


def _pair(B, Hq, Hkv, L, D, seed, softcap=0.0, v_fmt=mxfa.FMT_E4M3):
    """(noalloc O, workspace O, params, host operands) for one decode problem."""
    print(f"noalloc decode B{B} Hq{Hq} Hkv{Hkv} L{L} D{D} seed {seed}", flush=True)
    fp, dev, host = gen_qkv(B, Hq, Hkv, 1, L, D, seed, v_fmt=v_fmt)
    p = mxfa.make_params(B, Hq, Hkv, 1, L, D, causal=True, q_pos0=L - 1, softcap=softcap, v_fmt=v_fmt)
    _, ws = mxfa.decode_plan(p)
    assert ws <= mxfa.DECODE_SCRATCH_BYTES
    ops = [dev[n] for n in ("q", "qs", "k", "ks", "v", "vs")]
    got = torch.full((B, Hq, 1, D), float("nan"), dtype=torch.float32, device=DEV)
    L_ = mxfa.lib()
    st = L_.mxfa_decode_noalloc(ctypes.byref(p), *[ctypes.c_void_p(t.data_ptr()) for t in ops],
                                ctypes.c_void_p(got.data_ptr()),
                                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, L_.mxfa_last_error()
    want = mxfa.decode(p, *ops)
    torch.cuda.synchronize()
    return got, want, p, host


@pytest.mark.parametrize("big,small", [
    ((2, 32, 1, 1024, 128, 61), (1, 32, 1, 512, 128, 62)),               # group 32: combine kernel
    ((2, 16, 8, 2080, 256, 63), (1, 16, 8, 1056, 256, 64)),              # D = 256: combine kernel
    ((4, 32, 8, 1024, 128, 65), (2, 32, 8, 544, 128, 66)),               # merge inside the workgroup
])
def test_noalloc_matches_workspace_decode(big, small):
    mxfa.init()
    for B, Hq, Hkv, L, D, seed in (big, small):
        got, want, p, host = _pair(B, Hq, Hkv, L, D, seed, softcap=30.0 if D == 256 else 0.0)
        assert bool(torch.isfinite(got).all())
        assert torch.equal(got, want)
        n_parts, _ = mxfa.decode_plan(p)
        ref = O.attention(oracle_params(p), host["q"], host["qs"], host["k"], host["ks"], host["v"], host["vs"],
                          block_n=mxfa.DEFAULT_BLOCK_N, n_parts=n_parts)
        rel, mab = errors(np_(got), ref)
        print(f"   n_parts {n_parts} rel-L2 {rel:.3e} max-abs {mab:.3e}", flush=True)
        assert rel <= REL_L2_TOL and mab <= MAX_ABS_TOL
