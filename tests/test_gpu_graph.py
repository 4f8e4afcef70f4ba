"""HIP graph capture of the library's launches (serving loops capture their per-step work):
mxfa_prefill_ws (pre-pass + attention), mxfa_prefill, mxfa_decode with its partials
merged by the combine kernel, and mxfa_kv_append all launch on the caller's stream and
allocate or clear nothing, so they can be recorded into one graph.  The graph is replayed
several times with eager library work and synchronizations between the replays, and every
replay must reproduce the eager results bit for bit."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import mxfa  # noqa: E402
from gpuhelp import DEV, gen_qkv  # noqa: E402

pytestmark = pytest.mark.gpu


def test_prefill_decode_append_replay_equal_eager(monkeypatch):
    mxfa.init()
    # the two-launch decode (partials in the workspace, then mxfa_decode_combine)
    monkeypatch.setenv("MXFA_DECODE_COMBINE", "kernel")
    # prefill: GQA causal D = 128 through the workspace form; Gemma-like D = 256 with
    # block-packed E3M2 V through the workspace-free form
    _, d1, _ = gen_qkv(1, 8, 2, 256, 256, 128, seed=700)
    p1 = mxfa.make_params(1, 8, 2, 256, 256, 128, causal=True)
    ws1 = torch.empty(mxfa.prefill_plan(p1), dtype=torch.uint8, device=DEV)
    f2, d2, _ = gen_qkv(1, 4, 2, 192, 192, 256, seed=701, v_fmt=mxfa.FMT_E3M2)
    vb, vbs = mxfa.quantize_cols(f2["V"], mxfa.FMT_E3M2_BLK)
    p2 = mxfa.make_params(1, 4, 2, 192, 192, 256, causal=True, window=96, softcap=30.0, v_fmt=mxfa.FMT_E3M2_BLK)
    # decode over a 1,000-token cache
    _, d3, _ = gen_qkv(4, 16, 4, 1, 1024, 128, seed=702)
    p3 = mxfa.make_params(4, 16, 4, 1, 1024, 128, causal=True, q_pos0=999)
    _, ws3_bytes = mxfa.decode_plan(p3)
    ws3 = torch.empty(ws3_bytes, dtype=torch.uint8, device=DEV)
    # append of 40 tokens (two blocks touched, the second left open) into a fresh cache
    rng = np.random.default_rng(703)
    kn = torch.from_numpy(rng.standard_normal((2, 2, 40, 64)).astype(np.float32)).to(DEV)
    vn = torch.from_numpy(rng.standard_normal((2, 2, 40, 64)).astype(np.float32)).to(DEV)

    o1 = torch.empty((1, 8, 256, 128), dtype=torch.float32, device=DEV)
    o2 = torch.empty((1, 4, 192, 256), dtype=torch.float32, device=DEV)
    o3 = torch.empty((4, 16, 1, 128), dtype=torch.float32, device=DEV)
    cache = mxfa.KvCache(2, 2, 64, 128)

    def work():
        mxfa.prefill(p1, d1["q"], d1["qs"], d1["k"], d1["ks"], d1["v"], d1["vs"], out=o1, workspace=ws1)
        mxfa.prefill(p2, d2["q"], d2["qs"], d2["k"], d2["ks"], vb, vbs, out=o2, workspace=False)
        mxfa.decode(p3, d3["q"], d3["qs"], d3["k"], d3["ks"], d3["v"], d3["vs"], out=o3, workspace=ws3)
        cache.length = 0
        cache.append(kn, vn)

    # eager reference (on a side stream, as the capture will be)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        work()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    want = [t.clone() for t in (o1, o2, o3, cache.k, cache.ks, cache.v, cache.vs, cache.tail)]

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        work()
    for rep in range(3):
        print(f"replay {rep}", flush=True)
        for t in (o1, o2, o3):
            t.fill_(float("nan"))
        for t in (cache.k, cache.ks, cache.v, cache.vs, cache.tail):
            t.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = (o1, o2, o3, cache.k, cache.ks, cache.v, cache.vs, cache.tail)
        for i, (a, b) in enumerate(zip(got, want)):
            assert torch.equal(a, b), (rep, i)
        # eager library work between the replays, into other buffers
        mxfa.prefill(p1, d1["q"], d1["qs"], d1["k"], d1["ks"], d1["v"], d1["vs"], workspace=False)
        mxfa.decode(p3, d3["q"], d3["qs"], d3["k"], d3["ks"], d3["v"], d3["vs"])
        torch.cuda.synchronize()
