"""Benchmark: MXFP8 flash attention on one MI355X.

Headline (BASELINE.json metric "MXFP8 attn TFLOP/s + % MFMA peak (S=4096 GQA); decode
KV GB/s, 1 GPU"): a step is one mxfa_prefill_ws call (its bf16 K pass and the attention
kernel, workspace allocated once before timing) over configs[2] -- B=2, Hq=32, Hkv=8,
S=4096, D=128, causal, E4M3 block-32 MX operands with 1% of elements x20.
Operands are generated and quantized on the GPU before timing and stay resident in
HBM.  value = algorithmic TFLOP/s (4*D FLOP per visible (query, key) pair).  The
decode config is timed the same way and reported as HBM GB/s.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-decode]

Prints one JSON line.  Only --gpus 1 is supported (this path runs on one GPU).
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "radiance-kernels_amd"))

MXFP8_PEAK_TFLOPS = 5000.0     # MI355X dense fp8 / MXFP8 MFMA
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E


def prefill_config():
    return dict(B=2, Hq=32, Hkv=8, S=4096, D=128, causal=True, outlier_p=0.01)


def decode_config():
    return dict(B=64, Hq=32, Hkv=8, L=8192, D=128)


# The other prefill configs of BASELINE.json (timed for the roofline table; the headline is
# configs[2]).  N(0,1) inputs; c4 is the gemma variant (window, softcap, E3M2 V), timed with V
# block-packed (FMT_E3M2_BLK: the same E3M2 codes and scales, stored as the MFMA's fp6 operand)
# and, as c4_e3m2_bytes, with the codes one per byte.
OTHER_CONFIGS = {
    "c1": dict(B=1, Hq=1, Hkv=1, S=256, D=64, causal=False, outlier_p=0.0),
    "c2": dict(B=4, Hq=16, Hkv=16, S=2048, D=128, causal=True, outlier_p=0.0),
    "c4": dict(B=1, Hq=16, Hkv=8, S=8192, D=256, causal=True, outlier_p=0.0, window=4096, softcap=50.0,
               v_fmt=2),                                            # mxfa.FMT_E3M2_BLK
    "c4_e3m2_bytes": dict(B=1, Hq=16, Hkv=8, S=8192, D=256, causal=True, outlier_p=0.0, window=4096, softcap=50.0,
                          v_e3m2=True),
}


def make_prefill(torch, mxfa, c, seed=1):
    dev = "cuda:0"
    Q = torch.empty((c["B"], c["Hq"], c["S"], c["D"]), dtype=torch.float32, device=dev)
    K = torch.empty((c["B"], c["Hkv"], c["S"], c["D"]), dtype=torch.float32, device=dev)
    V = torch.empty_like(K)
    for i, X in enumerate((Q, K, V)):
        mxfa.fill_normal(X, seed * 3 + i, c["outlier_p"], 20.0)
    vf = c.get("v_fmt", mxfa.FMT_E3M2 if c.get("v_e3m2") else mxfa.FMT_E4M3)
    q, qs = mxfa.quantize_rows(Q)
    k, ks = mxfa.quantize_rows(K)
    v, vs = mxfa.quantize_cols(V, vf)
    del Q, K, V
    p = mxfa.make_params(c["B"], c["Hq"], c["Hkv"], c["S"], c["S"], c["D"], causal=c["causal"],
                         window=c.get("window", 0), softcap=c.get("softcap", 0.0), v_fmt=vf)
    return p, (q, qs, k, ks, v, vs)


def bench_other_configs(torch, mxfa, args):
    """configs[0], [1], [3]: TFLOP/s of mxfa_prefill_ws and the roofline fraction max(F/P_mfma,
    B/BW_hbm) / t, B = codes + scales read once + fp32 O written once (E3M2 V counted at 6
    bits); the workspace-free entry point (mxfa_prefill) timed beside it."""
    res = {}
    for name, c in OTHER_CONFIGS.items():
        p, ops = make_prefill(torch, mxfa, c, seed=7)
        out = torch.empty((p.batch, p.num_q_heads, p.seq_q, p.head_dim), dtype=torch.float32, device="cuda:0")
        ws = prefill_workspace(torch, mxfa, p)
        ms = time_calls(torch, lambda: mxfa.prefill(p, *ops, out=out, workspace=ws), max(20, args.steps // 4),
                        args.warmup)
        # the workspace-free entry point (mxfa_prefill) on the same operands
        ms_nw = time_calls(torch, lambda: mxfa.prefill(p, *ops, out=out, workspace=False), max(20, args.steps // 4),
                           args.warmup)
        flops = mxfa.attention_flops(p)
        vbytes = ops[4].numel() * (0.75 if p.v_fmt == mxfa.FMT_E3M2 else 1.0)   # block-packed: 6 bits already
        nbytes = sum(t.numel() for t in (ops[0], ops[1], ops[2], ops[3], ops[5])) + vbytes + out.numel() * 4
        t = ms * 1e-3
        frac = max(flops / (MXFP8_PEAK_TFLOPS * 1e12), nbytes / (HBM_PEAK_GBS * 1e9)) / t
        res[name] = {"shape": f"B={c['B']} Hq={c['Hq']} Hkv={c['Hkv']} S={c['S']} D={c['D']}"
                              + (" causal" if c["causal"] else "") + (f" window={c['window']}" if c.get("window") else "")
                              + (f" softcap={c['softcap']}" if c.get("softcap") else "") + {mxfa.FMT_E3M2: " V=E3M2", mxfa.FMT_E3M2_BLK: " V=E3M2 block-packed"}.get(p.v_fmt, ""),
                     "ms_per_call": round(ms, 4), "tflops": round(flops / t / 1e12, 1),
                     "workspace_free": {"ms_per_call": round(ms_nw, 4), "tflops": round(flops / (ms_nw * 1e-3) / 1e12, 1)},
                     "gflop": round(flops / 1e9, 3), "mb": round(nbytes / 1e6, 1), "roofline_frac": round(frac, 4),
                     "mfma_ceiling": round(mfma_ceiling(mxfa, p, flops)[0], 4)}
        del ops, out, ws
    return res


def prefill_workspace(torch, mxfa, p):
    """The caller workspace of mxfa_prefill_ws (bf16 K copy), allocated once."""
    return torch.empty(max(mxfa.prefill_plan(p), 16), dtype=torch.uint8, device="cuda:0")


def hbm_copy_gbs(torch):
    """Measured device-to-device copy rate (read + write bytes per second), 1 GiB."""
    n = 1 << 30
    a = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    b = torch.empty_like(a)
    a.fill_(1)
    ms = time_calls(torch, lambda: b.copy_(a), 20, 3)
    del a, b
    return round(2 * n / (ms * 1e-3) / 1e9, 1)


PREHEAT_S = 0.25


def time_calls(torch, fn, steps, warmup, preheat=True):
    """Average ms per call with HIP events on the launch stream (torch's current stream).
    Untimed before the K timed calls: the W warmup calls, then more calls until at least
    PREHEAT_S seconds of them have run -- the shader clock needs about that long under load
    to settle (measured: a 10-call warmup of the prefill kernel left the timed calls ~12%
    slower than steady state)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.time()
    while preheat and time.time() - t0 < PREHEAT_S:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        fn()
    ev1.record()
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / steps


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "prefill_c3_hbm_traffic.txt")
# the device sources the code object is built from, hashed in this order
KERNEL_SOURCES = [os.path.join(ROOT, "radiance-kernels_amd", "csrc", f)
                  for f in ("mxfa_kernels.hip", "kernel_base.h", "k_quant.hip", "k_attn_common.hip", "k_prefill.hip",
                            "k_decode.hip", "k_gemm.hip", "mx_device.h", "e3m2_rule.h", "mxfa_args.h", "log2_table.h")]


def kernel_source_sha():
    """sha256 (first 16 hex digits) of the device sources the code object is built from
    (concatenated in KERNEL_SOURCES order)."""
    import hashlib
    h = hashlib.sha256()
    for path in KERNEL_SOURCES:
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def profile_fields(path, keys):
    """key: value lines of a committed rocprofv3 summary (None when absent)."""
    out = dict.fromkeys(keys)
    try:
        with open(path) as f:
            for line in f:
                k, _, v = line.partition(":")
                if k in out:
                    out[k] = v.strip()
    except OSError:
        pass
    return out


def measured_traffic():
    """HBM bytes per prefill step from the committed rocprofv3 --pmc summary (FETCH_SIZE and
    WRITE_SIZE of both launches of a call, each scaled by its plain-copy calibration factor):
    {"step": bytes, "attention": bytes, "prepass": bytes, "source": ..., "kernel_source_sha":
    sha of the profiled source, "current": whether it is the source of this build}, or None."""
    f = profile_fields(TRAFFIC_PROFILE, ("traffic_bytes_per_step", "traffic_bytes_per_launch",
                                         "prepass_traffic_bytes", "kernel_source_sha256"))
    if f["traffic_bytes_per_launch"] is None:
        return None
    att = int(f["traffic_bytes_per_launch"])
    pre = int(f["prepass_traffic_bytes"]) if f["prepass_traffic_bytes"] else None
    step = int(f["traffic_bytes_per_step"]) if f["traffic_bytes_per_step"] else (att + (pre or 0))
    return {"step": step, "attention": att, "prepass": pre, "source": "profiles/prefill_c3_hbm_traffic.txt",
            "kernel_source_sha": f["kernel_source_sha256"],
            "current": f["kernel_source_sha256"] == kernel_source_sha()}


COUNTERS_PROFILE = os.path.join(ROOT, "profiles", "prefill_c3_counters.txt")


def measured_mfma_busy():
    """MFMA-busy % of the configs[2] attention kernel from the committed rocprofv3 --pmc summary
    (SQ_VALU_MFMA_BUSY_CYCLES over SQ_BUSY_CYCLES x 1024 SIMDs) -- not measured in this run --
    with the sha of the kernel source it was profiled from and whether that is this build's."""
    f = profile_fields(COUNTERS_PROFILE, ("mfma_busy_pct", "kernel_source_sha256"))
    if f["mfma_busy_pct"] is None:
        return None
    return {"pct": float(f["mfma_busy_pct"]), "source": "committed profile profiles/prefill_c3_counters.txt "
            "(rocprofv3 --pmc; not measured in this run)", "kernel": "mxfa_prefill3_d128",
            "kernel_source_sha": f["kernel_source_sha256"], "current": f["kernel_source_sha256"] == kernel_source_sha()}


# MFMA clocks per wave-block (32 queries x 64 keys) of the workspace prefill: D/16 x 2 score
# MFMAs v_mfma_f32_32x32x16_bf16 (32 clocks each) and D/32 PV MFMAs
# v_mfma_scale_f32_32x32x64_f8f6f4 (64 clocks each); 1,024 SIMDs at the 2.4 GHz clock the
# 5.0 PFLOP/s MXFP8 peak is quoted at.
PEAK_CLOCK_HZ = 2.4e9
# the shader clock the c3 prefill holds under load: its SQ_BUSY_CYCLES over its launch time
LOADED_CLOCK_HZ = 2.0e9
SIMDS = 1024


def prefill3_wave_blocks(mxfa, p):
    """Wave-blocks one mxfa_prefill_ws call runs: every wave of a workgroup walks the
    workgroup's key blocks [j0, j1) (the kernel's loop bounds; masked or not)."""
    group = p.num_q_heads // p.num_kv_heads
    hpw = next(h for h in (4, 2, 1) if group % h == 0)
    qpw = 32 * (4 // hpw)
    n_qblk = -(-p.seq_q // qpw)
    nkb = -(-p.seq_k // mxfa.DEFAULT_BLOCK_N)
    per_head_group = 0
    for qblk in range(n_qblk):
        q0 = qblk * qpw
        qmax = min(q0 + qpw, p.seq_q) - 1
        j0 = max(0, p.q_pos0 + q0 - p.window + 1) // mxfa.DEFAULT_BLOCK_N if p.window > 0 else 0
        j1 = min(nkb, max(0, p.q_pos0 + qmax) // mxfa.DEFAULT_BLOCK_N + 1) if p.causal else nkb
        per_head_group += 4 * max(0, j1 - j0)
    return per_head_group * p.batch * p.num_kv_heads * (group // hpw)


def mfma_ceiling(mxfa, p, flops):
    """The roofline fraction the kernel could reach with its MFMA pipes 100% busy: algorithmic
    FLOP over the time its MFMA instructions alone take, at the peak's clock."""
    D = p.head_dim
    clocks = prefill3_wave_blocks(mxfa, p) * ((D // 16) * 2 * 32 + (D // 32) * 64)
    t = clocks / SIMDS / PEAK_CLOCK_HZ
    return flops / t / (MXFP8_PEAK_TFLOPS * 1e12), clocks


def calibrate_copy(torch):
    """A plain device-to-device copy of known size, for scaling the FETCH_SIZE / WRITE_SIZE
    counters (run under rocprofv3 --pmc)."""
    n = 256 * 1024 * 1024
    a = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    b = torch.empty_like(a)
    a.fill_(1)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "device copy", "bytes_per_copy": n, "copies": 3}), flush=True)


def bench_decode_d256(torch, mxfa, args):
    """Decode at configs[3]'s head shape (Gemma-like: Hq 16, Hkv 8, D 256, softcap 50) over a
    batch of 32 caches of 8,192 tokens, V as E4M3 and as block-packed E3M2.  Bytes = codes and
    scales of Q, K, V read + fp32 O written."""
    dev = "cuda:0"
    B, Hq, Hkv, L, D = 32, 16, 8, 8192, 256
    Q = torch.empty((B, Hq, 1, D), dtype=torch.float32, device=dev)
    X = torch.empty((B, Hkv, L, D), dtype=torch.float32, device=dev)
    mxfa.fill_normal(Q, 21)
    mxfa.fill_normal(X, 22)
    q, qs = mxfa.quantize_rows(Q)
    k, ks = mxfa.quantize_rows(X)
    mxfa.fill_normal(X, 23)
    vs_ = {fmt: mxfa.quantize_cols(X, fmt) for fmt in (mxfa.FMT_E4M3, mxfa.FMT_E3M2_BLK)}
    del X
    o = torch.empty((B, Hq, 1, D), dtype=torch.float32, device=dev)
    out = {"workload": f"decode B={B} Hq={Hq} Hkv={Hkv} D={D} KV length {L}, softcap 50"}
    for key, fmt in (("v_e4m3", mxfa.FMT_E4M3), ("v_e3m2_blk", mxfa.FMT_E3M2_BLK)):
        v, vsc = vs_[fmt]
        p = mxfa.make_params(B, Hq, Hkv, 1, L, D, causal=True, q_pos0=L - 1, softcap=50.0, v_fmt=fmt)
        _, wsb = mxfa.decode_plan(p)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        ms = time_calls(torch, lambda: mxfa.decode(p, q, qs, k, ks, v, vsc, out=o, workspace=ws),
                        args.steps * 5, args.warmup)
        nb = sum(t.numel() for t in (q, qs, k, ks, v, vsc)) + o.numel() * 4
        out[key] = {"ms_per_call": round(ms, 4), "bytes_per_call": nb, "value": round(nb / (ms * 1e-3) / 1e9, 1),
                    "unit": "GB/s"}
    return out


def bench_kv_append(torch, mxfa, args):
    """KV-cache append (mxfa_kv_append): a 4096-token prefill chunk into a configs[2]-shape
    cache (B=2, Hkv=8, D=128) and a one-token decode step into a configs[4]-shape cache
    (B=64, Hkv=8, D=128, position 8191, whose open V block is re-quantized from the fp32
    tail).  Bytes = fp32 tokens read + codes/scales written + tail read/written."""
    dev = "cuda:0"
    out = {}
    for name, (B, H, D, L, pos, n) in {"prefill_4096": (2, 8, 128, 4096, 0, 4096),
                                       "decode_step": (64, 8, 128, 8192, 8191, 1)}.items():
        cache = mxfa.KvCache(B, H, D, L)
        kn = torch.empty((B, H, n, D), dtype=torch.float32, device=dev)
        vn = torch.empty_like(kn)
        mxfa.fill_normal(kn, 21)
        mxfa.fill_normal(vn, 22)

        def call():
            cache.length = pos
            cache.append(kn, vn)
        ms = time_calls(torch, call, args.steps, args.warmup)
        # the one-token step's call rate above is set by the Python wrapper's host time; its
        # device time: 100 calls captured in one HIP graph and replayed (each replay repeats the
        # same append, so the cache ends as after one)
        dev_ms = None
        if n == 1:
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                call()
            torch.cuda.current_stream().wait_stream(s)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(100):
                    call()
            graph.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            best = float("inf")
            for _ in range(5):
                e0.record()
                graph.replay()
                e1.record()
                torch.cuda.synchronize()
                best = min(best, e0.elapsed_time(e1) / 100)
            dev_ms = best
            del graph
        tok_in = 2 * B * H * n * D * 4
        blocks = (pos + n - 1) // 32 - pos // 32 + 1
        codes = B * H * (n * D + n * D // 32 + blocks * 32 * D + blocks * D)
        tail = B * H * 32 * D * 4 * ((1 if pos % 32 else 0) + (1 if (pos + n) % 32 else 0))   # read + write
        nbytes = tok_in + codes + tail
        out[name] = {"workload": f"B={B} Hkv={H} D={D}, {n} token(s) at position {pos}", "ms_per_call": round(ms, 4),
                     "bytes_per_call": nbytes, "value": round(nbytes / (ms * 1e-3) / 1e9, 1), "unit": "GB/s"}
        if dev_ms is not None:
            out[name]["graph_replay"] = {"ms_per_call": round(dev_ms, 4), "value": round(nbytes / (dev_ms * 1e-3) / 1e9, 1),
                                         "unit": "GB/s", "note": "100 appends in one HIP graph: device time, no host calls"}
    return out


def bench_gemm(torch, mxfa, args):
    """MX GEMM (mxfa_gemm) on the QKV projection of configs[2]: tokens M = B * S = 8192,
    hidden K = Hq * D = 4096, N = (Hq + 2 Hkv) * D = 6144, E4M3 activations and weights
    quantized on the GPU.  FLOP = 2 M N K."""
    dev = "cuda:0"
    M, K, N = 8192, 4096, 6144
    X = torch.empty((M, K), dtype=torch.float32, device=dev)
    W = torch.empty((K, N), dtype=torch.float32, device=dev)
    mxfa.fill_normal(X, 41)
    mxfa.fill_normal(W, 42)
    xq, xs = mxfa.quantize_rows(X)
    wq, ws = mxfa.quantize_cols(W)
    xs = xs.t().contiguous()
    del X, W
    c = torch.empty((M, N), dtype=torch.float32, device=dev)
    ms = time_calls(torch, lambda: mxfa.gemm(xq, xs, wq, ws, out=c), args.steps, args.warmup)
    tflops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    del c
    c16 = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    ms16 = time_calls(torch, lambda: mxfa.gemm(xq, xs, wq, ws, out=c16, c_fmt=mxfa.C_BF16), args.steps, args.warmup)
    tf16 = 2.0 * M * N * K / (ms16 * 1e-3) / 1e12
    # the same weights at decode batch M = 64 (the skinny kernel: one workgroup per 32-column
    # strip); HBM-bound on the weights, so reported as the weight stream rate
    Md = 64
    Xd = torch.empty((Md, K), dtype=torch.float32, device=dev)
    mxfa.fill_normal(Xd, 43)
    xdq, xds = mxfa.quantize_rows(Xd)
    xds = xds.t().contiguous()
    cd = torch.empty((Md, N), dtype=torch.float32, device=dev)
    msd = time_calls(torch, lambda: mxfa.gemm(xdq, xds, wq, ws, out=cd), args.steps, args.warmup)
    wbytes = wq.numel() + ws.numel()
    decode_m = {"workload": f"the same weights at decode batch M={Md} (N={N} K={K})", "ms_per_call": round(msd, 4),
                "weight_bytes": wbytes, "value": round(wbytes / (msd * 1e-3) / 1e9, 1), "unit": "GB/s",
                "frac_hbm_peak": round(wbytes / (msd * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    del Xd, xdq, xds, cd
    return {"workload": f"QKV projection of configs[2]: M={M} N={N} K={K}, E4M3 x E4M3 -> fp32",
            "value": round(tflops, 1), "unit": "TFLOP/s", "ms_per_call": round(ms, 4),
            "frac_mxfp8_peak": round(tflops / MXFP8_PEAK_TFLOPS, 4),
            "bf16_out": {"value": round(tf16, 1), "unit": "TFLOP/s", "ms_per_call": round(ms16, 4),
                         "frac_mxfp8_peak": round(tf16 / MXFP8_PEAK_TFLOPS, 4)},
            "decode_batch": decode_m}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# Host threads of the CPU baseline: every core this process may run on, up to the 16 host
# threads that one GPU's share of the GPU box comes with (the box runs other GPUs' jobs on
# the rest, whatever the cpu count reports).
CPU_THREAD_CAP = 16


def cpu_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(n, CPU_THREAD_CAP)), n


ORACLE_NATIVE_FLAGS = ["-O3", "-march=native", "-ffp-contract=off", "-fPIC", "-shared", "-std=c11", "-D_GNU_SOURCE"]


def native_oracle():
    """The CPU oracle compiled on this host with -march=native (the baseline build the plan
    names), into a temporary directory; (path, flags) or (None, reason) when no compiler runs."""
    import subprocess
    import tempfile
    d = tempfile.mkdtemp(prefix="mxfa_oracle_")
    out = os.path.join(d, "liboracle_native.so")
    cmd = [os.environ.get("CC", "gcc")] + ORACLE_NATIVE_FLAGS + ["-o", out, os.path.join(ROOT, "oracle", "mx_oracle.c"),
                                                                 "-lm", "-lpthread"]
    try:
        subprocess.run(cmd, check=True, capture_output=True, timeout=120)
        return out, " ".join(ORACLE_NATIVE_FLAGS)
    except (OSError, subprocess.SubprocessError) as e:
        return None, f"native build failed ({e.__class__.__name__}); the prebuilt -O3 oracle ran instead"


def cpu_baseline(mxfa, p, ops_host, threads, visible):
    """The CPU oracle (this repo's C restatement of the reference algorithm, threaded over
    query heads) on the whole configs[2] workload: every (batch, query head), the same
    block size.  About 40 thread-seconds of CPU work.  Built here with -O3 -march=native."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    lib_path, flags = native_oracle()
    if lib_path:
        O.LIB_PATH = lib_path
    op = O.make_params(p.batch, p.num_q_heads, p.num_kv_heads, p.seq_q, p.seq_k, p.head_dim,
                       causal=bool(p.causal), scale=p.softmax_scale)
    t0 = time.time()
    O.attention(op, *ops_host, block_n=mxfa.DEFAULT_BLOCK_N, nthreads=threads)
    dt = time.time() - t0
    flops = mxfa.attention_flops(p)
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "cpus_visible": visible, "build": flags,
            "sample": f"all of configs[2]: {p.batch} x {p.num_q_heads} query heads ({flops / 1e9:.1f} GFLOP, "
                      f"{dt:.2f} s wall on {threads} threads of {visible} visible; the GPU box gives one GPU "
                      f"{CPU_THREAD_CAP} host threads)"}


def profile_workload(torch, mxfa, name, args):
    """Run one workload alone, for rocprofv3: W untimed calls, then K calls timed with HIP
    events on the launch stream.  Prints one JSON line."""
    dev = "cuda:0"
    if name in ("c3", "c3r2"):
        p, ops = make_prefill(torch, mxfa, prefill_config())
        if name == "c3r2":
            p.p_rule = mxfa.P_R2
    elif name in OTHER_CONFIGS:
        p, ops = make_prefill(torch, mxfa, OTHER_CONFIGS[name], seed=7)
    elif name in ("decode", "decode256"):
        # decode256: bench_decode_d256's shape (Hq 16, Hkv 8, D 256, softcap 50, B 32, L 8192)
        dc = decode_config() if name == "decode" else dict(B=32, Hq=16, Hkv=8, L=8192, D=256)
        cap = 0.0 if name == "decode" else 50.0
        Qd = torch.empty((dc["B"], dc["Hq"], 1, dc["D"]), dtype=torch.float32, device=dev)
        Kd = torch.empty((dc["B"], dc["Hkv"], dc["L"], dc["D"]), dtype=torch.float32, device=dev)
        mxfa.fill_normal(Qd, 11)
        mxfa.fill_normal(Kd, 12)
        qd, qsd = mxfa.quantize_rows(Qd)
        kd, ksd = mxfa.quantize_rows(Kd)
        mxfa.fill_normal(Kd, 13)
        vd, vsd = mxfa.quantize_cols(Kd)
        del Kd
        pd = mxfa.make_params(dc["B"], dc["Hq"], dc["Hkv"], 1, dc["L"], dc["D"], causal=True, q_pos0=dc["L"] - 1,
                              softcap=cap)
        _, ws_bytes = mxfa.decode_plan(pd)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        od = torch.empty((dc["B"], dc["Hq"], 1, dc["D"]), dtype=torch.float32, device=dev)
        ms = time_calls(torch, lambda: mxfa.decode(pd, qd, qsd, kd, ksd, vd, vsd, out=od, workspace=ws),
                        args.steps, args.warmup, preheat=False)
        print(json.dumps({"profile": name, "ms_per_call": round(ms, 4), "calls": args.steps + args.warmup}), flush=True)
        return
    elif name in ("gemm", "gemm64"):
        # bench_gemm's QKV projection, fp32 C; gemm64: the same weights at decode batch M = 64
        M, K, N = (8192 if name == "gemm" else 64), 4096, 6144
        X = torch.empty((M, K), dtype=torch.float32, device=dev)
        W = torch.empty((K, N), dtype=torch.float32, device=dev)
        mxfa.fill_normal(X, 41)
        mxfa.fill_normal(W, 42)
        xq, xs = mxfa.quantize_rows(X)
        wq, ws = mxfa.quantize_cols(W)
        xs = xs.t().contiguous()
        del X, W
        c = torch.empty((M, N), dtype=torch.float32, device=dev)
        ms = time_calls(torch, lambda: mxfa.gemm(xq, xs, wq, ws, out=c), args.steps, args.warmup, preheat=False)
        print(json.dumps({"profile": name, "ms_per_call": round(ms, 4), "calls": args.steps + args.warmup,
                          "tflops": round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 1)}), flush=True)
        return
    else:
        raise SystemExit(f"bench.py: unknown --profile workload {name!r}")
    out = torch.empty((p.batch, p.num_q_heads, p.seq_q, p.head_dim), dtype=torch.float32, device=dev)
    ws = prefill_workspace(torch, mxfa, p)
    ms = time_calls(torch, lambda: mxfa.prefill(p, *ops, out=out, workspace=ws), args.steps, args.warmup,
                    preheat=False)
    flops = mxfa.attention_flops(p)
    print(json.dumps({"profile": name, "ms_per_call": round(ms, 4), "calls": args.steps + args.warmup,
                      "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true", help="only run a 256 MiB device copy x3")
    ap.add_argument("--profile", metavar="WORKLOAD",
                    help="run one workload alone for rocprofv3 (c1, c2, c3, c3r2, c4, decode, decode256, gemm, gemm64): W untimed + K timed calls")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU; --gpus must be 1 (the path is not sharded across GPUs here)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    torch.cuda.set_device(0)
    if args.calibrate_copy:
        calibrate_copy(torch)
        return
    import mxfa
    mxfa.init()
    if args.profile:
        profile_workload(torch, mxfa, args.profile, args)
        return

    c = prefill_config()
    p, ops = make_prefill(torch, mxfa, c)
    out = torch.empty((p.batch, p.num_q_heads, p.seq_q, p.head_dim), dtype=torch.float32, device="cuda:0")
    ws = prefill_workspace(torch, mxfa, p)
    ms = time_calls(torch, lambda: mxfa.prefill(p, *ops, out=out, workspace=ws), args.steps, args.warmup)
    flops = mxfa.attention_flops(p)
    tflops = flops / (ms * 1e-3) / 1e12

    result = {
        "metric": "MXFP8 attn TFLOP/s + % MFMA peak (S=4096 GQA); decode KV GB/s, 1 GPU",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "preheat_s": PREHEAT_S,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp8-e4m3 (QK^T on bf16 MFMA from exact dequant, PV on scaled MXFP8 MFMA, fp32 softmax/accum)",
        "data": "synthetic: N(0,1) with 1% of elements x20, generated and MX-quantized on the GPU (mxfa_fill_normal, mxfa_quantize_*)",
        "config": {"workload": "configs[2]: MXFP8 GQA causal prefill B=2 Hq=32 Hkv=8 S=4096 D=128",
                   "batch": c["B"], "q_heads": c["Hq"], "kv_heads": c["Hkv"], "seq": c["S"], "head_dim": c["D"],
                   "causal": True, "block_n": mxfa.DEFAULT_BLOCK_N, "gflop_per_step": round(flops / 1e9, 2)},
        "pct_mxfp8_peak": round(100.0 * tflops / MXFP8_PEAK_TFLOPS, 2),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": MXFP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MXFP8_PEAK_TFLOPS, 4), "traffic": None},
        "mfma_busy_from_profile": measured_mfma_busy(),
    }
    tr = measured_traffic()
    if tr is not None:
        result["roofline"]["traffic"] = tr["step"]
        result["roofline"]["traffic_detail"] = tr
    ceil, clocks = mfma_ceiling(mxfa, p, flops)
    result["roofline"]["mfma_ceiling"] = round(ceil, 4)
    result["roofline"]["mfma_ceiling_basis"] = (
        f"{clocks / 1e6:.1f} M SIMD-clocks of MFMA per step ({prefill3_wave_blocks(mxfa, p)} wave-blocks x "
        f"{(p.head_dim // 16) * 64 + (p.head_dim // 32) * 64} clocks: bf16 QK^T + MXFP8 PV) over {SIMDS} SIMDs at "
        f"{PEAK_CLOCK_HZ / 1e9:.1f} GHz; 0.5 of peak needs the MFMA pipes {50.0 / ceil:.0f}% busy at that clock, "
        f"{50.0 / ceil * PEAK_CLOCK_HZ / LOADED_CLOCK_HZ:.0f}% at the ~{LOADED_CLOCK_HZ / 1e9:.1f} GHz the shader clock "
        f"holds under this load (SQ_BUSY_CYCLES over the launch time)")

    # the same workload with the reference device kernels' P rule (R2 compatibility mode)
    p2 = mxfa.make_params(p.batch, p.num_q_heads, p.num_kv_heads, p.seq_q, p.seq_k, p.head_dim, causal=True,
                          p_rule=mxfa.P_R2)
    ms2 = time_calls(torch, lambda: mxfa.prefill(p2, *ops, out=out, workspace=ws), args.steps, args.warmup)
    result["prefill_p_rule_r2"] = {"workload": "configs[2] with P rule R2 (bf16 P, truncating target-0 requant)",
                                   "value": round(flops / (ms2 * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
                                   "ms_per_call": round(ms2, 4)}

    if not args.no_decode:
        dc = decode_config()
        dev = "cuda:0"
        Qd = torch.empty((dc["B"], dc["Hq"], 1, dc["D"]), dtype=torch.float32, device=dev)
        Kd = torch.empty((dc["B"], dc["Hkv"], dc["L"], dc["D"]), dtype=torch.float32, device=dev)
        mxfa.fill_normal(Qd, 11)
        mxfa.fill_normal(Kd, 12)
        qd, qsd = mxfa.quantize_rows(Qd)
        kd, ksd = mxfa.quantize_rows(Kd)
        mxfa.fill_normal(Kd, 13)
        vd, vsd = mxfa.quantize_cols(Kd)
        # the same V as MXFP6 E3M2, codes one per byte and block-packed
        v3, v3s = mxfa.quantize_cols(Kd, mxfa.FMT_E3M2)
        vb, vbs = mxfa.quantize_cols(Kd, mxfa.FMT_E3M2_BLK)
        del Kd
        pd = mxfa.make_params(dc["B"], dc["Hq"], dc["Hkv"], 1, dc["L"], dc["D"], causal=True, q_pos0=dc["L"] - 1)
        _, ws_bytes = mxfa.decode_plan(pd)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        od = torch.empty((dc["B"], dc["Hq"], 1, dc["D"]), dtype=torch.float32, device=dev)
        msd = time_calls(torch, lambda: mxfa.decode(pd, qd, qsd, kd, ksd, vd, vsd, out=od, workspace=ws),
                         args.steps * 5, args.warmup)
        nbytes = sum(t.numel() for t in (qd, qsd, kd, ksd, vd, vsd)) + od.numel() * 4
        gbs = nbytes / (msd * 1e-3) / 1e9
        result["decode"] = {"workload": "configs[4]: decode B=64 Hq=32 Hkv=8 D=128 KV length 8192, E4M3 MX KV cache",
                            "value": round(gbs, 1), "unit": "GB/s", "ms_per_call": round(msd, 4),
                            "bytes_per_call": nbytes, "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        # E3M2 V at the same shape: bytes moved per call with the codes one per byte and with
        # them block-packed (6 bits, read by the MFMA as they are)
        for key, fmt, vv, vvs in (("v_e3m2_bytes", mxfa.FMT_E3M2, v3, v3s), ("v_e3m2_blk", mxfa.FMT_E3M2_BLK, vb, vbs)):
            pv = mxfa.make_params(dc["B"], dc["Hq"], dc["Hkv"], 1, dc["L"], dc["D"], causal=True, q_pos0=dc["L"] - 1,
                                  v_fmt=fmt)
            msv = time_calls(torch, lambda: mxfa.decode(pv, qd, qsd, kd, ksd, vv, vvs, out=od, workspace=ws),
                             args.steps * 5, args.warmup)
            nbv = sum(t.numel() for t in (qd, qsd, kd, ksd, vv, vvs)) + od.numel() * 4
            result["decode"][key] = {"ms_per_call": round(msv, 4), "bytes_per_call": nbv,
                                     "value": round(nbv / (msv * 1e-3) / 1e9, 1), "unit": "GB/s"}
        del v3, v3s, vb, vbs

    if not args.no_decode:
        result["decode"]["hbm_copy_gbs"] = hbm_copy_gbs(torch)
        result["decode"]["d256"] = bench_decode_d256(torch, mxfa, args)
        result["kv_append"] = bench_kv_append(torch, mxfa, args)
        result["gemm"] = bench_gemm(torch, mxfa, args)
        result["other_configs"] = bench_other_configs(torch, mxfa, args)
    props = torch.cuda.get_device_properties(0)
    result["device"] = {"name": props.name, "arch": getattr(props, "gcnArchName", ""),
                        "compute_units": props.multi_processor_count,
                        "memory_gib": round(props.total_memory / 2 ** 30, 1)}

    if not args.no_cpu:
        threads, visible = cpu_threads()
        host = [t.cpu().numpy() for t in ops]
        result["cpu_baseline"] = cpu_baseline(mxfa, p, host, threads, visible)

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
