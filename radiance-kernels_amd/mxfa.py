"""Python host mirror of the libmxfa C ABI (include/mxfa.h).

The reference exposes its MXFP8 flash-attention operator as generated headers plus a
bare-metal entry point (kernels/flash_attention_mx_gqa/fa_gen_data.py:119-159,
kernel.cpp:91-191); its Python side (flash_attention_model.py) names the operations
make_inputs / mx_quantize_cols / mx_attention_flash*.  This module keeps that
vocabulary on top of the C ABI:

    fill_normal       -> make_inputs / make_inputs_gqa (synthetic N(0,1) [+ outliers])
    quantize_rows     -> mx_quantize_cols on Q and K (32-blocks along D)
    quantize_cols     -> mx_quantize_cols(V.t()) (32-blocks along the key axis)
    quantize_rows_r4  -> the simt_quant block quantizer (rule R4)
    prefill           -> mx_attention_flash[_causal_gqa | _gemma]
    decode            -> the same recurrence over an MXFP8 KV cache (split-KV)
    softmax_requant   -> fused_softmax_requant (the P tile step, for bit-exact checks)
    KvCache.append    -> the producer side of decode: new tokens into the MXFP8 cache

torch is used only to hold device memory and name the stream; every call goes through
ctypes into libmxfa.so, which launches gfx950 kernels.  There is no fallback: if the
library or the code object is missing, calls raise.
"""
import ctypes
import math
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmxfa.so")

FMT_E4M3 = 0
FMT_E3M2 = 1
FMT_E3M2_BLK = 2    # E3M2 V packed per 32-row MX block: [..., rows/32, cols, 24] bytes (the MFMA fp6 operand)
P_R1 = 0        # P requant rule of lib/golden (default)
P_R2 = 1        # the reference device kernels' truncating "target-0" rule
DEFAULT_BLOCK_N = 64

STATUS = {0: "ok", 1: "invalid argument", 2: "unsupported", 3: "HIP error", 4: "code object error",
          5: "workspace too small"}


class MxfaError(RuntimeError):
    def __init__(self, status, detail):
        self.status = status
        super().__init__(f"mxfa: {STATUS.get(status, status)}: {detail}")


class AttnParams(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32), ("num_q_heads", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32),
        ("seq_q", ctypes.c_int32), ("seq_k", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("causal", ctypes.c_int32), ("q_pos0", ctypes.c_int32), ("window", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float), ("softcap", ctypes.c_float), ("v_fmt", ctypes.c_int32),
        ("block_n", ctypes.c_int32), ("p_rule", ctypes.c_int32), ("kv_stride", ctypes.c_int32),
    ]


def make_params(B, Hq, Hkv, Sq, Sk, D, causal=False, q_pos0=0, window=0, scale=None, softcap=0.0,
                v_fmt=FMT_E4M3, block_n=0, p_rule=P_R1, kv_stride=0):
    return AttnParams(B, Hq, Hkv, Sq, Sk, D, int(bool(causal)), int(q_pos0), int(window),
                      float(scale if scale is not None else 1.0 / math.sqrt(D)), float(softcap), int(v_fmt),
                      int(block_n), int(p_rule), int(kv_stride))


def _need(t, dtype, shape, name):
    """Device, dtype, layout and shape check of one operand before its pointer is passed
    on (the kernels read through raw pointers: a host, short or strided tensor would be
    read out of bounds)."""
    import torch
    if not (isinstance(t, torch.Tensor) and t.is_cuda):
        raise MxfaError(1, f"{name} must be a CUDA tensor")
    if t.dtype != dtype:
        raise MxfaError(1, f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise MxfaError(1, f"{name} must be contiguous")
    if tuple(t.shape) != tuple(shape):
        raise MxfaError(1, f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")


def _check_attn_operands(p, q, qs, k, ks, v, vs, out):
    import torch
    B, Hq, Hkv, Sq, D = p.batch, p.num_q_heads, p.num_kv_heads, p.seq_q, p.head_dim
    L = p.kv_stride or p.seq_k
    u8 = torch.uint8
    _need(q, u8, (B, Hq, Sq, D), "q")
    _need(qs, u8, (B, Hq, Sq, D // 32), "q_sc")
    _need(k, u8, (B, Hkv, L, D), "k")
    _need(ks, u8, (B, Hkv, L, D // 32), "k_sc")
    _need(v, u8, (B, Hkv, L // 32, D, 24) if p.v_fmt == FMT_E3M2_BLK else (B, Hkv, L, D), "v")
    _need(vs, u8, (B, Hkv, L // 32, D), "v_sc")
    _need(out, torch.float32, (B, Hq, Sq, D), "out")


class KvParams(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("max_len", ctypes.c_int32), ("v_fmt", ctypes.c_int32)]


C_F32, C_BF16 = 0, 1                    # mxfa_c_fmt


class GemmParams(ctypes.Structure):
    _fields_ = [("m", ctypes.c_int64), ("n", ctypes.c_int64), ("k", ctypes.c_int64),
                ("a_fmt", ctypes.c_int32), ("b_fmt", ctypes.c_int32), ("c_fmt", ctypes.c_int32)]


EXPORTS = ("mxfa_quantize_rows", "mxfa_quantize_rows_r4", "mxfa_quantize_cols", "mxfa_prefill", "mxfa_prefill_plan",
           "mxfa_prefill_ws", "mxfa_prefill_trace", "mxfa_decode_plan", "mxfa_decode", "mxfa_decode_noalloc",
           "mxfa_kv_append", "mxfa_softmax_requant", "mxfa_fill_normal", "mxfa_init", "mxfa_shutdown", "mxfa_status_string",
           "mxfa_last_error", "mxfa_version", "mxfa_gemm")

_lib = None


def lib():
    """Load libmxfa.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MxfaError(4, f"{LIB_PATH} not built (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        vp, u8p, f32p = ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p
        P = ctypes.POINTER
        L.mxfa_quantize_rows.argtypes = [f32p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int, u8p, u8p, vp]
        L.mxfa_quantize_cols.argtypes = [f32p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int, u8p, u8p, vp]
        L.mxfa_quantize_rows_r4.argtypes = [f32p, ctypes.c_int64, ctypes.c_int32, u8p, u8p, vp]
        L.mxfa_prefill.argtypes = [P(AttnParams)] + [u8p] * 6 + [f32p, vp]
        L.mxfa_prefill_plan.argtypes = [P(AttnParams), P(ctypes.c_size_t)]
        L.mxfa_prefill_ws.argtypes = [P(AttnParams)] + [u8p] * 6 + [f32p, vp, ctypes.c_size_t, vp]
        L.mxfa_prefill_trace.argtypes = ([P(AttnParams)] + [u8p] * 6 + [f32p, vp, ctypes.c_size_t, ctypes.c_int32,
                                         ctypes.c_int32, f32p, f32p, u8p, u8p, vp])
        L.mxfa_decode_plan.argtypes = [P(AttnParams), P(ctypes.c_int32), P(ctypes.c_size_t)]
        L.mxfa_decode.argtypes = [P(AttnParams)] + [u8p] * 6 + [f32p, vp, ctypes.c_size_t, vp]
        L.mxfa_decode_noalloc.argtypes = [P(AttnParams)] + [u8p] * 6 + [f32p, vp]
        L.mxfa_softmax_requant.argtypes = [f32p, f32p, ctypes.c_float, ctypes.c_int64, ctypes.c_int32,
                                           ctypes.c_int32, f32p, u8p, u8p, f32p, vp]
        L.mxfa_fill_normal.argtypes = [f32p, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_float, vp]
        L.mxfa_kv_append.argtypes = [P(KvParams), f32p, f32p, ctypes.c_int32, ctypes.c_int32] + [u8p] * 4 + [f32p, vp]
        L.mxfa_gemm.argtypes = [P(GemmParams), u8p, u8p, u8p, u8p, vp, vp]
        L.mxfa_status_string.argtypes = [ctypes.c_int]
        L.mxfa_status_string.restype = ctypes.c_char_p
        L.mxfa_last_error.restype = ctypes.c_char_p
        L.mxfa_version.restype = ctypes.c_int32
        for name in ("mxfa_quantize_rows", "mxfa_quantize_rows_r4", "mxfa_quantize_cols", "mxfa_prefill",
                     "mxfa_prefill_plan", "mxfa_prefill_ws", "mxfa_prefill_trace", "mxfa_decode_plan", "mxfa_decode",
                     "mxfa_decode_noalloc", "mxfa_softmax_requant", "mxfa_fill_normal", "mxfa_init", "mxfa_kv_append", "mxfa_gemm"):
            getattr(L, name).restype = ctypes.c_int
        _lib = L
    return _lib


def _check(st):
    if st != 0:
        raise MxfaError(st, lib().mxfa_last_error().decode())


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(stream):
    if stream is None:
        import torch
        # the raw handle of torch's current stream on the current device, read without building
        # a Stream object (a few microseconds per call, which short kernels such as the
        # decode-batch GEMM would otherwise wait on)
        raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
        if raw is not None:
            return ctypes.c_void_p(raw(torch._C._cuda_getDevice()))
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return ctypes.c_void_p(stream if isinstance(stream, int) else stream.cuda_stream)


def init():
    _check(lib().mxfa_init())


def quantize_rows(x, fmt=FMT_E4M3, stream=None):
    """x: contiguous float32 CUDA tensor [..., cols] -> (codes uint8 [..., cols], scales uint8 [..., cols/32])."""
    import torch
    assert x.is_cuda and x.dtype == torch.float32 and x.is_contiguous()
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    codes = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    scales = torch.empty(tuple(x.shape[:-1]) + (cols // 32,), dtype=torch.uint8, device=x.device)
    _check(lib().mxfa_quantize_rows(_ptr(x), rows, cols, fmt, _ptr(codes), _ptr(scales), _stream(stream)))
    return codes, scales


def quantize_rows_r4(x, stream=None):
    """Rule R4 (the reference's simt_quant block quantizer), 32-blocks along the last axis."""
    import torch
    assert x.is_cuda and x.dtype == torch.float32 and x.is_contiguous()
    cols = x.shape[-1]
    rows = x.numel() // cols
    codes = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    scales = torch.empty(tuple(x.shape[:-1]) + (cols // 32,), dtype=torch.uint8, device=x.device)
    _check(lib().mxfa_quantize_rows_r4(_ptr(x), rows, cols, _ptr(codes), _ptr(scales), _stream(stream)))
    return codes, scales


def quantize_cols(x, fmt=FMT_E4M3, stream=None):
    """x: contiguous float32 CUDA tensor [..., rows, cols]; 32-blocks along rows ->
    (codes [..., rows, cols] (FMT_E3M2_BLK: [..., rows/32, cols, 24]), scales [..., rows/32, cols])."""
    import torch
    assert x.is_cuda and x.dtype == torch.float32 and x.is_contiguous()
    rows, cols = x.shape[-2], x.shape[-1]
    mats = x.numel() // (rows * cols)
    cshape = tuple(x.shape[:-2]) + (rows // 32, cols, 24) if fmt == FMT_E3M2_BLK else x.shape
    codes = torch.empty(cshape, dtype=torch.uint8, device=x.device)
    scales = torch.empty(tuple(x.shape[:-2]) + (rows // 32, cols), dtype=torch.uint8, device=x.device)
    _check(lib().mxfa_quantize_cols(_ptr(x), mats, rows, cols, fmt, _ptr(codes), _ptr(scales), _stream(stream)))
    return codes, scales


# Block-packed E3M2: rows 8g + 4a + b (g < 4, a < 2, b < 4) of a 32-row block sit at 6-bit
# field 16a + 4g + b, i.e. the group of four rows 4q .. 4q + 3 fills bytes 3u .. 3u + 2 with
# u = 4 (q % 2) + q // 2 -- the key order in which the attention kernels' P operand meets the
# MFMA's fp6 V operand.
_BLK_UNIT_GROUP = [2 * (u % 4) + u // 4 for u in range(8)]      # 3-byte unit u <- row group q
_BLK_GROUP_UNIT = [4 * (q % 2) + q // 2 for q in range(8)]      # row group q -> 3-byte unit u


def blk_field(r):
    """6-bit field of row r (0..31) in a block-packed E3M2 block."""
    return 16 * ((r >> 2) & 1) + 4 * (r >> 3) + (r & 3)


def e3m2_to_blk(codes):
    """Host (numpy) repacking of E3M2 codes one per byte, [..., rows, cols] with rows % 32 == 0,
    into the FMT_E3M2_BLK layout [..., rows/32, cols, 24]: row r of a 32-row block in bits
    6f .. 6f+5, f = blk_field(r), of its column's 24 bytes read as a 192-bit little-endian
    integer."""
    import numpy as np
    c = np.asarray(codes, dtype=np.uint8)
    *lead, rows, cols = c.shape
    c = (c & 0x3F).reshape(*lead, rows // 32, 8, 4, cols)[..., _BLK_UNIT_GROUP, :, :]
    c = np.moveaxis(c, -1, -3).astype(np.uint32)                        # [..., rows/32, cols, unit, 4]
    w = c[..., 0] | (c[..., 1] << 6) | (c[..., 2] << 12) | (c[..., 3] << 18)
    out = np.stack([w & 0xFF, (w >> 8) & 0xFF, (w >> 16) & 0xFF], axis=-1).astype(np.uint8)
    return out.reshape(*lead, rows // 32, cols, 24)


def e3m2_from_blk(blk):
    """Inverse of e3m2_to_blk: [..., nb, cols, 24] -> E3M2 codes one per byte [..., 32 nb, cols]."""
    import numpy as np
    b = np.asarray(blk, dtype=np.uint8)
    *lead, nb, cols, _ = b.shape
    b = b.reshape(*lead, nb, cols, 8, 3).astype(np.uint32)[..., _BLK_GROUP_UNIT, :]
    w = b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16)
    c = np.stack([(w >> (6 * i)) & 0x3F for i in range(4)], axis=-1)   # [..., nb, cols, group, 4]
    c = np.moveaxis(c.reshape(*lead, nb, cols, 32), -2, -1)            # [..., nb, 32, cols]
    return c.reshape(*lead, nb * 32, cols).astype(np.uint8)


def softmax_requant(s, row_max, c, p_rule=P_R1, stream=None):
    """The kernels' softmax-requant step on scores s [..., cols] (cols % 32 == 0) with
    per-row maxima row_max [...] under P rule p_rule: returns (p, codes, scales, row_sum)
    (mxfa_softmax_requant)."""
    import torch
    assert s.is_cuda and s.dtype == torch.float32 and s.is_contiguous()
    assert row_max.is_cuda and row_max.dtype == torch.float32 and row_max.is_contiguous()
    cols = s.shape[-1]
    rows = s.numel() // cols
    assert row_max.numel() == rows
    p = torch.empty_like(s)
    codes = torch.empty(s.shape, dtype=torch.uint8, device=s.device)
    scales = torch.empty(tuple(s.shape[:-1]) + (cols // 32,), dtype=torch.uint8, device=s.device)
    row_sum = torch.empty(tuple(s.shape[:-1]), dtype=torch.float32, device=s.device)
    _check(lib().mxfa_softmax_requant(_ptr(s), _ptr(row_max), float(c), rows, cols, int(p_rule), _ptr(p),
                                      _ptr(codes), _ptr(scales), _ptr(row_sum), _stream(stream)))
    return p, codes, scales, row_sum


def gemm(a, a_sc, b, b_sc, a_fmt=FMT_E4M3, b_fmt=FMT_E4M3, out=None, stream=None, c_fmt=C_F32):
    """MX GEMM (mxfa_gemm): a [M][K] and b [K][N] uint8 codes, a_sc [K/32][M] and
    b_sc [K/32][N] E8M0 codes (CUDA tensors) -> C [M][N] float32 (c_fmt C_F32) or
    bfloat16 (C_BF16)."""
    import torch
    M, K = a.shape
    N = b.shape[1]
    for t in (a, a_sc, b, b_sc):
        assert t.is_cuda and t.dtype == torch.uint8 and t.is_contiguous()
    assert b.shape[0] == K and tuple(a_sc.shape) == (K // 32, M) and tuple(b_sc.shape) == (K // 32, N)
    dt = torch.bfloat16 if c_fmt == C_BF16 else torch.float32
    if out is None:
        out = torch.empty((M, N), dtype=dt, device=a.device)
    assert out.dtype == dt and out.is_contiguous() and tuple(out.shape) == (M, N)
    p = GemmParams(M, N, K, int(a_fmt), int(b_fmt), int(c_fmt))
    _check(lib().mxfa_gemm(ctypes.byref(p), _ptr(a), _ptr(a_sc), _ptr(b), _ptr(b_sc), _ptr(out), _stream(stream)))
    return out


def fill_normal(x, seed, outlier_p=0.0, outlier_mul=20.0, stream=None):
    """Fill a contiguous float32 CUDA tensor with N(0,1) values (+ outliers) in place."""
    import torch
    assert x.is_cuda and x.dtype == torch.float32 and x.is_contiguous()
    _check(lib().mxfa_fill_normal(_ptr(x), x.numel(), ctypes.c_uint64(seed & (2 ** 64 - 1)), float(outlier_p),
                                  float(outlier_mul), _stream(stream)))
    return x


def prefill_plan(p):
    """Workspace bytes of mxfa_prefill_ws for p: the bf16 copy of K (B * Hkv * Sk * D * 2
    bytes), plus the E4M3 copy of V (B * Hkv * Sk * D bytes) when V is FMT_E3M2 (block-packed
    FMT_E3M2_BLK V is read as it is).  Never 0."""
    ws = ctypes.c_size_t(0)
    _check(lib().mxfa_prefill_plan(ctypes.byref(p), ctypes.byref(ws)))
    return ws.value


def prefill(p, q, qs, k, ks, v, vs, out=None, workspace=None, stream=None):
    """O [B, Hq, Sq, D] fp32 of MXFP8 attention; operands in the C-ABI layouts (k/v/k_sc/v_sc
    with p.kv_stride keys per (batch, KV head) when it is set).  workspace: None allocates
    prefill_plan(p) bytes and calls mxfa_prefill_ws; a uint8 CUDA tensor is passed to
    mxfa_prefill_ws; False calls mxfa_prefill (no workspace)."""
    import torch
    if out is None:
        out = torch.empty((p.batch, p.num_q_heads, p.seq_q, p.head_dim), dtype=torch.float32, device=q.device)
    _check_attn_operands(p, q, qs, k, ks, v, vs, out)
    args = (ctypes.byref(p), _ptr(q), _ptr(qs), _ptr(k), _ptr(ks), _ptr(v), _ptr(vs), _ptr(out))
    if workspace is False:
        _check(lib().mxfa_prefill(*args, _stream(stream)))
        return out
    if workspace is None:
        workspace = torch.empty(max(prefill_plan(p), 16), dtype=torch.uint8, device=q.device)
    _need(workspace, torch.uint8, (workspace.numel(),), "workspace")
    _check(lib().mxfa_prefill_ws(*args, _ptr(workspace), workspace.numel(), _stream(stream)))
    return out


def prefill_trace(p, q, qs, k, ks, v, vs, bh, q_tile, stream=None):
    """Stages of the workspace prefill for query rows 32 * q_tile .. + 31 of head bh
    (mxfa_prefill_trace): dict of host arrays S [32][Sk] (kernel units, NaN where not
    written), m and l [n_blocks][32], codes [32][Sk] (0 where not written), scales
    [32][Sk/32], and the O of the call [B][Hq][Sq][D] (rows of this workgroup only)."""
    import torch
    dev = q.device
    Sk = p.seq_k
    nblk = (Sk + DEFAULT_BLOCK_N - 1) // DEFAULT_BLOCK_N
    out = torch.zeros((p.batch, p.num_q_heads, p.seq_q, p.head_dim), dtype=torch.float32, device=dev)
    _check_attn_operands(p, q, qs, k, ks, v, vs, out)
    ws = torch.empty(max(prefill_plan(p), 16), dtype=torch.uint8, device=dev)
    s_out = torch.full((32, Sk), float("nan"), dtype=torch.float32, device=dev)
    ml = torch.full((nblk, 32, 2), float("nan"), dtype=torch.float32, device=dev)
    codes = torch.zeros((32, Sk), dtype=torch.uint8, device=dev)
    scales = torch.zeros((32, Sk // 32), dtype=torch.uint8, device=dev)
    _check(lib().mxfa_prefill_trace(ctypes.byref(p), _ptr(q), _ptr(qs), _ptr(k), _ptr(ks), _ptr(v), _ptr(vs),
                                    _ptr(out), _ptr(ws), ws.numel(), int(bh), int(q_tile), _ptr(s_out), _ptr(ml),
                                    _ptr(codes), _ptr(scales), _stream(stream)))
    torch.cuda.synchronize()
    mlh = ml.cpu().numpy()
    return {"S": s_out.cpu().numpy(), "m": mlh[:, :, 0], "l": mlh[:, :, 1], "codes": codes.cpu().numpy(),
            "scales": scales.cpu().numpy(), "o": out}


def decode_plan(p):
    """(n_parts, workspace bytes): the decode's interleaved partials per head (partial i
    takes key blocks i, i + n_parts, ...) and the workspace mxfa.decode needs."""
    n = ctypes.c_int32(0)
    ws = ctypes.c_size_t(0)
    _check(lib().mxfa_decode_plan(ctypes.byref(p), ctypes.byref(n), ctypes.byref(ws)))
    return n.value, ws.value


def decode(p, q, qs, k, ks, v, vs, out=None, workspace=None, stream=None):
    import torch
    _, ws_bytes = decode_plan(p)
    if workspace is None:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    if out is None:
        out = torch.empty((p.batch, p.num_q_heads, 1, p.head_dim), dtype=torch.float32, device=q.device)
    _check_attn_operands(p, q, qs, k, ks, v, vs, out)
    _need(workspace, torch.uint8, (workspace.numel(),), "workspace")
    _check(lib().mxfa_decode(ctypes.byref(p), _ptr(q), _ptr(qs), _ptr(k), _ptr(ks), _ptr(v), _ptr(vs), _ptr(out),
                             _ptr(workspace), workspace.numel(), _stream(stream)))
    return out


DECODE_SCRATCH_BYTES = 16 << 20        # MXFA_DECODE_SCRATCH_BYTES


def decode_noalloc(p, q, qs, k, ks, v, vs, out, stream=None):
    """mxfa_decode_noalloc: decode with the partials in the library's per-device scratch
    (no workspace, nothing allocated by the call; out must be given)."""
    _check_attn_operands(p, q, qs, k, ks, v, vs, out)
    _check(lib().mxfa_decode_noalloc(ctypes.byref(p), _ptr(q), _ptr(qs), _ptr(k), _ptr(ks), _ptr(v), _ptr(vs),
                                     _ptr(out), _stream(stream)))
    return out


class KvCache:
    """An MXFP8 KV cache on the device (the layouts decode reads) plus the fp32 tail of
    its open V block; append() quantizes new tokens into it (mxfa_kv_append)."""

    def __init__(self, batch, num_kv_heads, head_dim, max_len, v_fmt=FMT_E4M3, device="cuda:0"):
        import torch
        B, H, D, L = batch, num_kv_heads, head_dim, max_len
        self.params = KvParams(B, H, D, L, v_fmt)
        self.k = torch.zeros((B, H, L, D), dtype=torch.uint8, device=device)
        self.ks = torch.zeros((B, H, L, D // 32), dtype=torch.uint8, device=device)
        vshape = (B, H, L // 32, D, 24) if v_fmt == FMT_E3M2_BLK else (B, H, L, D)
        self.v = torch.zeros(vshape, dtype=torch.uint8, device=device)
        self.vs = torch.zeros((B, H, L // 32, D), dtype=torch.uint8, device=device)
        self.tail = torch.zeros((B, H, 32, D), dtype=torch.float32, device=device)
        self.length = 0

    def decode_params(self, Hq, **kw):
        """mxfa_attn_params for decoding the next query over the cache as it stands: seq_k =
        length rounded up to 32, q_pos0 = length - 1 (the padding is masked causally),
        kv_stride = max_len (decode reads the cache tensors in place)."""
        P = self.params
        sk = (self.length + 31) // 32 * 32
        return make_params(P.batch, Hq, P.num_kv_heads, 1, sk, P.head_dim, causal=True, q_pos0=self.length - 1,
                           v_fmt=P.v_fmt, kv_stride=P.max_len, **kw)

    def append(self, k_new, v_new, stream=None):
        """k_new, v_new: contiguous float32 [B, Hkv, n_new, D] CUDA tensors."""
        import torch
        P = self.params
        n = k_new.shape[2] if k_new.dim() == 4 else -1
        _need(k_new, torch.float32, (P.batch, P.num_kv_heads, n, P.head_dim), "k_new")
        _need(v_new, torch.float32, (P.batch, P.num_kv_heads, n, P.head_dim), "v_new")
        if self.length + n > P.max_len:
            raise MxfaError(1, f"append of {n} tokens at {self.length} exceeds max_len {P.max_len}")
        _check(lib().mxfa_kv_append(ctypes.byref(self.params), _ptr(k_new), _ptr(v_new), self.length, n,
                                    _ptr(self.k), _ptr(self.ks), _ptr(self.v), _ptr(self.vs), _ptr(self.tail),
                                    _stream(stream)))
        self.length += n


def attention_flops(p):
    """Algorithmic FLOP of one call: 4*D per visible (query, key) pair (QK^T + PV)."""
    return 4.0 * p.head_dim * p.batch * p.num_q_heads * visible_pairs(p)


def visible_pairs(p):
    """Visible (query, key) pairs of one head under the causal / window mask."""
    total = 0
    for i in range(p.seq_q):
        qpos = p.q_pos0 + i
        hi = min(p.seq_k - 1, qpos) if p.causal else p.seq_k - 1
        lo = max(0, qpos - p.window + 1) if p.window > 0 else 0
        if hi >= lo:
            total += hi - lo + 1
    return total
