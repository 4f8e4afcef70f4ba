"""CPU tests of the C ABI: the library loads, exports every entry point declared in
include/mxfa.h, and rejects invalid arguments before touching a GPU."""
import ctypes
import os
import re

import pytest

import mxfa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    src = open(os.path.join(ROOT, "include", "mxfa.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(mxfa_[a-z_0-9]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    L = mxfa.lib()
    names = declared_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(L, n), n
    assert set(mxfa.EXPORTS) <= set(names)


def test_code_object_present_and_for_gfx950():
    path = os.path.join(os.path.dirname(mxfa.LIB_PATH), "mxfa_kernels.hsaco")
    data = open(path, "rb").read()
    assert data[:4] == b"\x7fELF" or data.startswith(b"__CLANG_OFFLOAD_BUNDLE__")
    assert b"gfx950" in data
    for k in ("mxfa_prefill3n_d256", "mxfa_decode_d128", "mxfa_quant_rows_e4m3", "mxfa_softmax_requant_rows",
              "mxfa_prefill3n_d128_softcap_r2_e3m2", "mxfa_decode_d64_softcap_r2", "mxfa_decode_scratch",
              "mxfa_k_to_bf16", "mxfa_prefill3_d128", "mxfa_prefill3_d64_softcap_r2", "mxfa_prefill3n_d128",
              "mxfa_prefill3_d256_softcap", "mxfa_prefill3n_d64"):
        assert k.encode() in data


def test_version_and_status_strings():
    L = mxfa.lib()
    assert L.mxfa_version() == 3
    assert L.mxfa_status_string(0) == b"ok"
    assert L.mxfa_status_string(5) == b"workspace too small"


def _call_prefill(p):
    L = mxfa.lib()
    buf = (ctypes.c_uint8 * 64)()
    ptr = ctypes.cast(ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16, ctypes.c_void_p)
    return L.mxfa_prefill(ctypes.byref(p), ptr, ptr, ptr, ptr, ptr, ptr, ptr, None)


@pytest.mark.parametrize("kw,status", [
    (dict(Hq=3, Hkv=2), 1),              # Hq % Hkv
    (dict(D=48), 1),                     # D % 32
    (dict(D=96), 2),                     # unsupported head dim
    (dict(Sk=100), 1),                   # Sk % 32
    (dict(B=0), 1),
    (dict(window=-1), 1),
    (dict(softcap=-1.0), 1),
    (dict(block_n=128), 2),
    (dict(p_rule=2), 1),
    (dict(p_rule=-1), 1),
    (dict(kv_stride=32), 1),             # below seq_k
    (dict(kv_stride=100), 1),            # not a multiple of 32
])
def test_prefill_argument_validation(kw, status):
    a = dict(B=1, Hq=2, Hkv=2, Sq=32, Sk=64, D=64, window=0, softcap=0.0, block_n=0, p_rule=0, kv_stride=0)
    a.update(kw)
    p = mxfa.make_params(a["B"], a["Hq"], a["Hkv"], a["Sq"], a["Sk"], a["D"], window=a["window"],
                         softcap=a["softcap"], block_n=a["block_n"], p_rule=a["p_rule"], kv_stride=a["kv_stride"])
    assert _call_prefill(p) == status
    assert mxfa.lib().mxfa_last_error()


def test_null_and_misaligned_pointers_rejected():
    L = mxfa.lib()
    p = mxfa.make_params(1, 1, 1, 32, 64, 64)
    assert L.mxfa_prefill(ctypes.byref(p), None, None, None, None, None, None, None, None) == 1
    buf = (ctypes.c_uint8 * 64)()
    base = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16
    mis = ctypes.c_void_p(base + 1)
    assert L.mxfa_prefill(ctypes.byref(p), mis, mis, mis, mis, mis, mis, mis, None) == 1


def test_decode_validation_and_plan():
    L = mxfa.lib()
    p = mxfa.make_params(64, 32, 8, 1, 8192, 128, causal=True, q_pos0=8191)
    nparts, ws = mxfa.decode_plan(p)
    assert nparts == 4                       # 2048 partial waves over 512 (b, KV head) pairs
    assert ws >= 64 * 32 * nparts * (128 + 2) * 4
    # small problems: at most one partial per 64-key block; 3 rounds up to 4
    assert mxfa.decode_plan(mxfa.make_params(1, 8, 8, 1, 128, 64, causal=True, q_pos0=127))[0] == 2
    assert mxfa.decode_plan(mxfa.make_params(1, 8, 1, 1, 64 * 40, 64, causal=True, q_pos0=2559))[0] == 40
    assert mxfa.decode_plan(mxfa.make_params(8, 32, 8, 1, 4096, 128, causal=True, q_pos0=4095))[0] == 32
    assert mxfa.decode_plan(mxfa.make_params(96, 32, 8, 1, 4096, 128, causal=True, q_pos0=4095))[0] == 4
    # D = 256 (one workgroup per CU): about 1,024 partial waves, half the D <= 128 target
    assert mxfa.decode_plan(mxfa.make_params(32, 16, 8, 1, 8192, 256, causal=True, q_pos0=8191))[0] == 4
    assert mxfa.decode_plan(mxfa.make_params(32, 16, 8, 1, 8192, 128, causal=True, q_pos0=8191))[0] == 8
    assert mxfa.decode_plan(mxfa.make_params(2, 16, 8, 1, 8192, 256, causal=True, q_pos0=8191))[0] == 64
    p2 = mxfa.make_params(1, 1, 1, 2, 64, 64)
    sl_ = ctypes.c_int32(0)
    ws_ = ctypes.c_size_t(0)
    assert L.mxfa_decode_plan(ctypes.byref(p2), ctypes.byref(sl_), ctypes.byref(ws_)) == 1


def test_quantize_argument_validation():
    L = mxfa.lib()
    assert L.mxfa_quantize_rows(None, 4, 48, 0, None, None, None) == 1
    assert L.mxfa_quantize_rows(None, 0, 64, 0, None, None, None) == 0     # empty input: no-op
    assert L.mxfa_quantize_cols(None, 1, 48, 64, 0, None, None, None) == 1
    assert L.mxfa_quantize_cols(None, 0, 64, 64, 0, None, None, None) == 0
    assert L.mxfa_softmax_requant(None, None, 1.0, 4, 33, 0, None, None, None, None, None) == 1
    assert L.mxfa_softmax_requant(None, None, 0.0, 4, 32, 0, None, None, None, None, None) == 1
    assert L.mxfa_softmax_requant(None, None, 1.0, 4, 32, 3, None, None, None, None, None) == 1   # bad rule
    assert L.mxfa_softmax_requant(None, None, 1.0, 0, 32, 1, None, None, None, None, None) == 0


def test_launches_past_2_pow_32_work_items_rejected_without_device():
    """A launch's x extent in work-items is a 32-bit count: calls that would need more are
    MXFA_ERR_UNSUPPORTED before any device work (the pointers are never touched)."""
    L = mxfa.lib()
    fake = ctypes.c_void_p(1 << 20)                       # aligned, never dereferenced
    big = 1 << 31
    assert L.mxfa_quantize_rows(fake, big, 32, 0, fake, fake, None) == 2
    assert b"2^32 work-items" in L.mxfa_last_error()
    assert L.mxfa_quantize_rows_r4(fake, big, 32, fake, fake, None) == 2
    assert L.mxfa_quantize_cols(fake, big, 32 * 1024, 128, 0, fake, fake, None) == 2
    assert L.mxfa_softmax_requant(fake, fake, 1.0, 1 << 33, 32, 0, fake, fake, fake, fake, None) == 2
    assert L.mxfa_fill_normal(fake, 1 << 33, 1, 0.0, 20.0, None) == 2
    kv = mxfa.KvParams(1 << 20, 64, 256, 1 << 20, mxfa.FMT_E4M3)
    assert L.mxfa_kv_append(ctypes.byref(kv), fake, fake, 0, 1 << 16, fake, fake, fake, fake, fake, None) == 2


def test_kv_append_argument_validation():
    L = mxfa.lib()
    P = mxfa.KvParams
    ok = P(2, 2, 128, 256, mxfa.FMT_E4M3)
    z = [None] * 6
    assert L.mxfa_kv_append(None, None, None, 0, 1, *z) == 1                       # no params
    assert L.mxfa_kv_append(ctypes.byref(ok), None, None, 0, 0, *z) == 0           # nothing to append
    assert L.mxfa_kv_append(ctypes.byref(ok), None, None, 0, 1, *z) == 1           # NULL buffers
    assert L.mxfa_kv_append(ctypes.byref(ok), None, None, 250, 7, *z) == 1         # past max_len
    assert L.mxfa_kv_append(ctypes.byref(ok), None, None, -1, 1, *z) == 1
    for bad in (P(2, 2, 100, 256, 0), P(2, 2, 128, 250, 0), P(0, 2, 128, 256, 0), P(2, 2, 128, 256, 7)):
        assert L.mxfa_kv_append(ctypes.byref(bad), None, None, 0, 1, *z) == 1


def test_quantize_r4_argument_validation():
    L = mxfa.lib()
    assert L.mxfa_quantize_rows_r4(None, 4, 48, None, None, None) == 1
    assert L.mxfa_quantize_rows_r4(None, 0, 64, None, None, None) == 0
    assert L.mxfa_quantize_rows_r4(None, 4, 64, None, None, None) == 1


def test_gemm_argument_validation():
    L = mxfa.lib()
    G = mxfa.GemmParams
    buf = (ctypes.c_uint8 * 64)()
    ptr = ctypes.cast(ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16, ctypes.c_void_p)
    for bad, status in ((G(0, 64, 64, 0, 0), 1), (G(64, 64, 48, 0, 0), 1), (G(64, 64, 96, 0, 0), 2),
                        (G(40, 64, 64, 0, 0), 2), (G(64, 64, 64, 3, 0), 1), (G(1 << 20, 64, 1 << 12, 0, 0), 2),
                        (G(64, 1 << 22, 64, 0, 0), 2), (G(64, 64, 64, 0, 0, 2), 1)):
        assert L.mxfa_gemm(ctypes.byref(bad), ptr, ptr, ptr, ptr, ptr, None) == status
    ok = G(64, 64, 64, 0, 0)
    assert L.mxfa_gemm(ctypes.byref(ok), None, ptr, ptr, ptr, ptr, None) == 1
    assert L.mxfa_gemm(None, ptr, ptr, ptr, ptr, ptr, None) == 1


def test_decode_noalloc_rejects_before_touching_the_device():
    """mxfa_decode_noalloc checks its arguments and the size of the partials against the
    16 MiB device scratch before any HIP call: an oversized shape is MXFA_ERR_WORKSPACE
    (the status is the same on a host without a GPU), NULL pointers MXFA_ERR_INVALID_ARG."""
    L = mxfa.lib()
    buf = (ctypes.c_uint8 * 64)()
    ptr = ctypes.c_void_p(ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16)
    big = mxfa.make_params(512, 64, 2, 1, 4096, 256, causal=True, q_pos0=4095)
    _, ws = mxfa.decode_plan(big)
    assert ws > mxfa.DECODE_SCRATCH_BYTES
    assert L.mxfa_decode_noalloc(ctypes.byref(big), ptr, ptr, ptr, ptr, ptr, ptr, ptr, None) == 5
    assert b"16777216-byte device scratch" in L.mxfa_last_error()
    ok = mxfa.make_params(64, 32, 8, 1, 8192, 128, causal=True, q_pos0=8191)
    assert mxfa.decode_plan(ok)[1] <= mxfa.DECODE_SCRATCH_BYTES
    assert L.mxfa_decode_noalloc(ctypes.byref(ok), None, None, None, None, None, None, None, None) == 1


def test_prefill_plan_and_workspace_checks():
    """mxfa_prefill_plan: the bf16 K copy (B * Hkv * Sk * D * 2 bytes), plus the E4M3 copy of
    an E3M2 V (B * Hkv * Sk * D bytes); mxfa_prefill_ws rejects a missing or short workspace
    with MXFA_ERR_WORKSPACE before touching the device."""
    L = mxfa.lib()
    p = mxfa.make_params(2, 32, 8, 4096, 4096, 128, causal=True)
    assert mxfa.prefill_plan(p) == 2 * 8 * 4096 * 128 * 2
    assert mxfa.prefill_plan(mxfa.make_params(1, 4, 2, 64, 4096, 64, kv_stride=8192)) == 2 * 4096 * 64 * 2
    assert mxfa.prefill_plan(mxfa.make_params(1, 16, 8, 128, 128, 256)) == 8 * 128 * 256 * 2
    assert mxfa.prefill_plan(mxfa.make_params(1, 4, 2, 64, 64, 128, v_fmt=mxfa.FMT_E3M2)) == 2 * 64 * 128 * 3
    assert L.mxfa_prefill_plan(ctypes.byref(p), None) == 1
    assert L.mxfa_prefill_plan(ctypes.byref(mxfa.make_params(1, 3, 2, 32, 64, 64)), ctypes.byref(ctypes.c_size_t())) == 1
    buf = (ctypes.c_uint8 * 64)()
    ptr = ctypes.c_void_p(ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16)
    small = mxfa.make_params(1, 2, 2, 32, 64, 64)
    need = mxfa.prefill_plan(small)
    assert L.mxfa_prefill_ws(ctypes.byref(small), *([ptr] * 7), None, need, None) == 5
    assert L.mxfa_prefill_ws(ctypes.byref(small), *([ptr] * 7), ptr, need - 1, None) == 5
    assert b"workspace needs" in L.mxfa_last_error()
    assert L.mxfa_prefill_ws(ctypes.byref(small), *([None] * 7), ptr, need, None) == 1


def test_kv_range_limit_rejected_without_device():
    """The kernels address one (batch, KV head) of K/V -- and the workspace's bf16 K, two
    bytes per element -- with 32-bit byte offsets: seq_k * head_dim * 2 must stay below 2^31.
    Shapes past it are MXFA_ERR_UNSUPPORTED at plan time (no device needed); the largest
    shape inside it is accepted."""
    L = mxfa.lib()
    ws = ctypes.c_size_t(0)
    for d in (64, 128, 256):
        limit = (2 ** 31 - 1) // (2 * d) // 32 * 32          # largest seq_k (multiple of 32) inside
        ok = mxfa.make_params(1, 1, 1, 1, limit, d)
        assert L.mxfa_prefill_plan(ctypes.byref(ok), ctypes.byref(ws)) == 0
        assert ws.value == limit * d * 2
        bad = mxfa.make_params(1, 1, 1, 1, limit + 32, d)
        assert L.mxfa_prefill_plan(ctypes.byref(bad), ctypes.byref(ws)) == 2
        assert b"32-bit K/V range" in L.mxfa_last_error()
        dec = mxfa.make_params(1, 1, 1, 1, limit + 32, d, causal=True, q_pos0=limit + 31)
        assert L.mxfa_decode_plan(ctypes.byref(dec), ctypes.byref(ctypes.c_int32()), ctypes.byref(ws)) == 2
