"""Operand-format adapter between the reference FA kernels' generated `fa_data.h` headers
and this library's tensor layouts.

The reference's FA "operator" takes its operands as C arrays in a generated header:

  GQA / Gemma kernels (kernels/flash_attention_mx_gqa/fa_gen_data.py:95-159,
  kernels/flash_attention_mx_gemma/fa_gen_data.py:122-200), head-major, only the
  FA_NBLK_USED leading key blocks (blocks_used, flash_attention_model.py:182-186):
    QK_A_in            [NQ*Sq][D]        Q codes, query head h at rows h*Sq
    QK_A_scales_row    [NQ*GK][Sq]       Q scales, transposed per head
    QK_B_blocks        [NKV*NBU*D][Bk]   K_j^T codes, block (kv*NBU + j) at rows (kv*NBU + j)*D
    QK_B_scales_blocks [NKV*NBU*GK][Bk]  K_j^T scales
    V_in               [NKV*NBU*Bk][D]   V codes, block (kv*NBU + j) at rows (kv*NBU + j)*Bk
    V_scales           [NKV*NBU*GKB][D]  V scales, 32-blocks along the key axis
  single-head kernels (kernels/flash_attention_mx/gen_data.py:73-128,
  kernels/flash_attention_mx_stable/gen_data.py:96-133), non-causal:
    QK_A_in [Sq][D], QK_B_in [D][Sk], QK_A_scales_row [GK][Sq], QK_B_scales_col [GK][Sk],
    V_in [Sk][D], V_scales [GKV][D], QK_B_blocks [NBLK*D][Bk], QK_B_scales_blocks [NBLK*GK][Bk]
  plus #define parameters (FA_SQ, FA_SK, FA_D, FA_BK, FA_NQ, FA_NKV, FA_QPOS0, ...).

This library takes q [B][Hq][Sq][D] + q_sc [B][Hq][Sq][D/32], k [B][Hkv][Sk][D] +
k_sc [B][Hkv][Sk][D/32], v [B][Hkv][Sk][D] + v_sc [B][Hkv][Sk/32][D].  export_fa_data()
converts one batch entry of ours to the reference arrays (and write_header() prints them
in the generator's text format); read_header() parses such a header and import_fa_data()
converts it back, zero-filling the key blocks the header leaves out (they lie above the
causal diagonal of every query, so they are masked and the attention result is the same).

Host-side numpy only (no GPU, no reference code): a format converter, not a kernel.
"""
import math
import re
from dataclasses import dataclass, field

import numpy as np

GROUP = 32
LAYOUTS = ("gqa", "gemma", "single")


def blocks_used(Sq, Sk, q_pos0, block_n):
    """Leading key blocks not entirely above the causal diagonal
    (kernels/flash_attention_mx_gqa/flash_attention_model.py:182-186)."""
    return min(Sk // block_n, (q_pos0 + Sq - 1) // block_n + 1)


def bf16_bits(x):
    """bf16 round-to-nearest-even bit pattern of a float (the generators' torch .to(bfloat16))."""
    b = int(np.array(x, np.float32).view(np.uint32))
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) & 0xFFFF


def bf16_value(bits):
    return float(np.array(int(bits) << 16, np.uint32).view(np.float32))


@dataclass
class FaData:
    """One reference operand set: the header's #defines and its arrays (numpy, 2-D)."""
    layout: str
    defines: dict = field(default_factory=dict)
    arrays: dict = field(default_factory=dict)


def _u8(a):
    return np.ascontiguousarray(np.asarray(a), dtype=np.uint8)


def export_fa_data(q, q_sc, k, k_sc, v, v_sc, *, block_n=64, q_pos0=0, layout="gqa", softcap=0.0, window=0,
                   batch_index=0, scale=None):
    """Our layouts (numpy uint8, batch dimension first) -> the reference arrays of one
    batch entry.  layout: "gqa" (causal), "gemma" (causal + softcap/window defines) or
    "single" (one head, non-causal, all key blocks).  scale: the softmax scale, written as
    FA_SOFTMAX_SCALE_BF16 (bf16, as the reference's header holds it); default 1/sqrt(D)."""
    if layout not in LAYOUTS:
        raise ValueError(f"layout must be one of {LAYOUTS}")
    q, q_sc, k, k_sc, v, v_sc = (_u8(a)[batch_index] for a in (q, q_sc, k, k_sc, v, v_sc))
    NQ, Sq, D = q.shape
    NKV, Sk, _ = k.shape
    Bk = block_n
    if D % GROUP or Sk % Bk or Bk % GROUP or NQ % NKV:
        raise ValueError("need D % 32 == 0, Sk % block_n == 0, block_n % 32 == 0, NQ % NKV == 0")
    if q_sc.shape != (NQ, Sq, D // GROUP) or k_sc.shape != (NKV, Sk, D // GROUP) or v.shape != (NKV, Sk, D) \
            or v_sc.shape != (NKV, Sk // GROUP, D):
        raise ValueError("operand shapes do not match the library layouts")
    GK, GKB, Nblk = D // GROUP, Bk // GROUP, Sk // Bk
    d = dict(FA_SQ=Sq, FA_SK=Sk, FA_D=D, FA_GK=GK, FA_GKV=Sk // GROUP, FA_BK=Bk, FA_NBLK=Nblk, FA_GKB=GKB)
    d["FA_SOFTMAX_SCALE_BF16"] = bf16_bits(1.0 / math.sqrt(D) if scale is None else scale)
    arr = {}
    if layout == "single":
        if NQ != 1 or NKV != 1:
            raise ValueError("the single-head layout holds one query head and one KV head")
        arr["QK_A_in"] = q[0]
        arr["QK_B_in"] = np.ascontiguousarray(k[0].T)
        arr["QK_A_scales_row"] = np.ascontiguousarray(q_sc[0].T)
        arr["QK_B_scales_col"] = np.ascontiguousarray(k_sc[0].T)
        arr["V_in"] = v[0]
        arr["V_scales"] = v_sc[0]
        arr["QK_B_blocks"] = np.ascontiguousarray(k[0].reshape(Nblk, Bk, D).transpose(0, 2, 1)).reshape(Nblk * D, Bk)
        arr["QK_B_scales_blocks"] = np.ascontiguousarray(
            k_sc[0].reshape(Nblk, Bk, GK).transpose(0, 2, 1)).reshape(Nblk * GK, Bk)
        return FaData(layout, d, arr)
    nbu = blocks_used(Sq, Sk, q_pos0, Bk)
    d.update(FA_NQ=NQ, FA_NKV=NKV, FA_GRP=NQ // NKV, FA_QPOS0=q_pos0, FA_NBLK_USED=nbu)
    if layout == "gemma":
        d.update(FA_ATTN_SOFTCAP=int(softcap > 0), FA_ATTN_SOFTCAP_BF16=bf16_bits(softcap) if softcap > 0 else 0x3C00,
                 FA_ATTN_SOFTCAP_INV_BF16=bf16_bits(1.0 / softcap) if softcap > 0 else 0x3C00,
                 FA_SLIDING=int(window > 0), FA_WINDOW=int(window))
    elif softcap or window:
        raise ValueError("softcap and window need the gemma layout")
    arr["QK_A_in"] = q.reshape(NQ * Sq, D)
    arr["QK_A_scales_row"] = np.ascontiguousarray(q_sc.transpose(0, 2, 1)).reshape(NQ * GK, Sq)
    kb = k[:, :nbu * Bk].reshape(NKV, nbu, Bk, D)
    ksb = k_sc[:, :nbu * Bk].reshape(NKV, nbu, Bk, GK)
    arr["QK_B_blocks"] = np.ascontiguousarray(kb.transpose(0, 1, 3, 2)).reshape(NKV * nbu * D, Bk)
    arr["QK_B_scales_blocks"] = np.ascontiguousarray(ksb.transpose(0, 1, 3, 2)).reshape(NKV * nbu * GK, Bk)
    arr["V_in"] = np.ascontiguousarray(v[:, :nbu * Bk]).reshape(NKV * nbu * Bk, D)
    arr["V_scales"] = np.ascontiguousarray(v_sc[:, :nbu * GKB]).reshape(NKV * nbu * GKB, D)
    return FaData(layout, d, arr)


def import_fa_data(fd, scale="header"):
    """Reference arrays -> (q, q_sc, k, k_sc, v, v_sc) in our layouts (batch 1) and the
    keyword arguments of mxfa.make_params for the same attention.  scale: "header" takes
    the softmax scale the reference device kernels compute with, the bf16
    FA_SOFTMAX_SCALE_BF16 (kernels/flash_attention_mx_gqa/kernel.cpp:52,149; 1/sqrt(128)
    is 0.08837890625 there); "fp32" takes 1/sqrt(D) as the reference's Python model does."""
    d, a = fd.defines, fd.arrays
    Sq, Sk, D, Bk = d["FA_SQ"], d["FA_SK"], d["FA_D"], d["FA_BK"]
    GK, GKB = D // GROUP, Bk // GROUP
    if scale == "header" and "FA_SOFTMAX_SCALE_BF16" in d:
        sc = float(np.array([d["FA_SOFTMAX_SCALE_BF16"] << 16], np.uint32).view(np.float32)[0])
    elif scale in ("header", "fp32"):
        sc = 1.0 / math.sqrt(D)
    else:
        raise ValueError('scale must be "header" or "fp32"')
    params = dict(B=1, Sq=Sq, Sk=Sk, D=D, scale=sc, block_n=Bk)
    if fd.layout == "single":
        q = a["QK_A_in"].reshape(1, 1, Sq, D)
        q_sc = np.ascontiguousarray(a["QK_A_scales_row"].T).reshape(1, 1, Sq, GK)
        k = np.ascontiguousarray(a["QK_B_in"].T).reshape(1, 1, Sk, D)
        k_sc = np.ascontiguousarray(a["QK_B_scales_col"].T).reshape(1, 1, Sk, GK)
        v = a["V_in"].reshape(1, 1, Sk, D)
        v_sc = a["V_scales"].reshape(1, 1, Sk // GROUP, D)
        params.update(Hq=1, Hkv=1, causal=False, q_pos0=0)
        return tuple(_u8(x) for x in (q, q_sc, k, k_sc, v, v_sc)), params
    NQ, NKV, nbu = d["FA_NQ"], d["FA_NKV"], d["FA_NBLK_USED"]
    q = a["QK_A_in"].reshape(1, NQ, Sq, D)
    q_sc = np.ascontiguousarray(a["QK_A_scales_row"].reshape(NQ, GK, Sq).transpose(0, 2, 1)).reshape(1, NQ, Sq, GK)
    k = np.zeros((1, NKV, Sk, D), np.uint8)
    k_sc = np.zeros((1, NKV, Sk, GK), np.uint8)
    v = np.zeros((1, NKV, Sk, D), np.uint8)
    v_sc = np.zeros((1, NKV, Sk // GROUP, D), np.uint8)
    k[0, :, :nbu * Bk] = a["QK_B_blocks"].reshape(NKV, nbu, D, Bk).transpose(0, 1, 3, 2).reshape(NKV, nbu * Bk, D)
    k_sc[0, :, :nbu * Bk] = a["QK_B_scales_blocks"].reshape(NKV, nbu, GK, Bk).transpose(0, 1, 3, 2).reshape(
        NKV, nbu * Bk, GK)
    v[0, :, :nbu * Bk] = a["V_in"].reshape(NKV, nbu * Bk, D)
    v_sc[0, :, :nbu * GKB] = a["V_scales"].reshape(NKV, nbu * GKB, D)
    params.update(Hq=NQ, Hkv=NKV, causal=True, q_pos0=d["FA_QPOS0"])
    if fd.layout == "gemma":
        if d.get("FA_ATTN_SOFTCAP", 0):
            params["softcap"] = bf16_value(d["FA_ATTN_SOFTCAP_BF16"])
        if d.get("FA_SLIDING", 0):
            params["window"] = d["FA_WINDOW"]
    return tuple(_u8(x) for x in (q, q_sc, k, k_sc, v, v_sc)), params


# ---------------------------------------------------------------- header text
_DIMS = {
    "gqa": {"QK_A_in": "[FA_NQ*FA_SQ][FA_D]", "QK_A_scales_row": "[FA_NQ*FA_GK][FA_SQ]",
            "QK_B_blocks": "[FA_NKV*FA_NBLK_USED*FA_D][FA_BK]",
            "QK_B_scales_blocks": "[FA_NKV*FA_NBLK_USED*FA_GK][FA_BK]",
            "V_in": "[FA_NKV*FA_NBLK_USED*FA_BK][FA_D]", "V_scales": "[FA_NKV*FA_NBLK_USED*FA_GKB][FA_D]"},
    "single": {"QK_A_in": "[FA_SQ][FA_D]", "QK_B_in": "[FA_D][FA_SK]", "QK_A_scales_row": "[FA_GK][FA_SQ]",
               "QK_B_scales_col": "[FA_GK][FA_SK]", "V_in": "[FA_SK][FA_D]", "V_scales": "[FA_GKV][FA_D]",
               "QK_B_blocks": "[FA_NBLK*FA_D][FA_BK]", "QK_B_scales_blocks": "[FA_NBLK*FA_GK][FA_BK]"},
}
_DIMS["gemma"] = _DIMS["gqa"]


def header_text(fd):
    """The header in the generators' format: #defines, then one `static const uint8_t
    NAME[..][..] = { { 0x.., ... }, ... };` per array (a 2-D initializer, one row per line)."""
    out = ["#ifndef FA_DATA_H", "#define FA_DATA_H", "", "#include <stdint.h>", ""]
    for name, val in fd.defines.items():
        out.append(f"#define {name} 0x{val:04x}" if name.endswith("_BF16") else f"#define {name} {val}")
    out.append("")
    for name, dims in _DIMS[fd.layout].items():
        a = fd.arrays[name]
        rows = ",\n".join("    { " + ", ".join(f"0x{int(x):02x}" for x in row) + " }" for row in a)
        out.append(f"static const uint8_t {name}{dims} = {{\n{rows}\n}};\n")
    out.append("#endif // FA_DATA_H")
    return "\n".join(out) + "\n"


def write_header(fd, path):
    with open(path, "w") as f:
        f.write(header_text(fd))


_DEF_RE = re.compile(r"^\s*#define\s+(FA_\w+)\s+(0x[0-9a-fA-F]+|-?\d+)\b", re.M)
_ARR_RE = re.compile(r"static\s+const\s+(uint8_t|uint16_t)\s+(\w+)\s*\[([^\]]+)\]\s*\[([^\]]+)\]\s*=\s*\{(.*?)\};", re.S)
_NUM_RE = re.compile(r"0x[0-9a-fA-F]+|\d+")


def _eval_dim(expr, defines):
    n = 1
    for term in expr.split("*"):
        term = term.strip()
        n *= defines[term] if term in defines else int(term, 0)
    return n


def read_header(text):
    """Parse a generated fa_data.h (text) into FaData.  The layout is "single" when the
    header has no FA_NQ, "gemma" when it has FA_ATTN_SOFTCAP, else "gqa".  Arrays the
    adapter does not use (bf16 goldens such as O_gold, QK_S_bf16) are parsed as well."""
    defines = {m.group(1): int(m.group(2), 0) for m in _DEF_RE.finditer(text)}
    arrays = {}
    for m in _ARR_RE.finditer(text):
        ctype, name, d0, d1, body = m.groups()
        rows, cols = _eval_dim(d0, defines), _eval_dim(d1, defines)
        vals = np.array([int(x, 0) for x in _NUM_RE.findall(body)], np.uint16 if ctype == "uint16_t" else np.uint8)
        if vals.size != rows * cols:
            raise ValueError(f"{name}: {vals.size} values for [{rows}][{cols}]")
        arrays[name] = vals.reshape(rows, cols)
    layout = "single" if "FA_NQ" not in defines else ("gemma" if "FA_ATTN_SOFTCAP" in defines else "gqa")
    return FaData(layout, defines, arrays)
