"""Write tests/golden/r4_blocks.npz: rule R4 (the reference's simt_quant block quantizer) on
blocks whose amax is tiny -- fp32 subnormals and the small normals below 2^-120, where the
reference builds its 2^-e multiplier from a 32-bit word (127 - e) << 23 that wraps -- and, for
contrast, blocks across the normal range and at amax = 448 * 2^k.

The expected outputs come from the reference's own bit primitives in lib/golden/golden.py
(block_exp, pow2_neg_e, fp8_code_rshift, f32_bits), imported from /root/reference and
composed per block as kernels/simt_quant/gen_quant.py:54-70 composes them (amax over the
block, e = block_exp(amax), scale code e + 127 clamped to [0, 254], element code =
fp8_code_rshift(x * pow2_neg_e(e)), an all-zero block gives scale 0 and codes 0).  That
composition is restated below because gen_quant.py writes into the reference tree when it
runs; golden.py itself only defines functions.

Run in the container that holds /root/reference:
    python tests/golden/make_r4_golden.py

Fixture (data only): x [blocks][32] float32 inputs, codes [blocks][32] uint8 E4M3 codes,
scales [blocks] uint8 E8M0 codes.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_GOLDEN = "/root/reference/lib/golden"


def inputs(rng):
    blocks = []
    # amax an fp32 subnormal: every binade 2^-149 .. 2^-127, random signs and mantissas,
    # the block's largest element at a random position
    for e in range(-149, -126):
        for _ in range(6):
            b = (rng.random(32) * 2.0 ** (e + 1)).astype(np.float32) * rng.choice([-1, 1], 32).astype(np.float32)
            b[rng.integers(32)] = np.float32(2.0 ** e) * np.float32(1.0 + rng.random())
            blocks.append(b)
    # the largest subnormal and the smallest normal as amax
    for a in (np.uint32(0x007fffff).view(np.float32), np.uint32(0x00800000).view(np.float32)):
        b = (rng.standard_normal(32) * 1e-40).astype(np.float32)
        b[0] = a
        blocks.append(b)
    # small normals up to 2^-100 (the multiplier's word wraps below about 2^-120)
    for e in range(-126, -99):
        for m in (1.0, 1.5, 1.75, 1.9999999):
            b = (rng.standard_normal(32) * 2.0 ** (e - 2)).astype(np.float32)
            b[rng.integers(32)] = np.float32(m * 2.0 ** e)
            blocks.append(b)
    # the normal range and amax at / next to 448 * 2^k
    for k in range(-60, 61, 3):
        base = np.float32(448.0 * 2.0 ** k)
        for a in (base, np.nextafter(base, np.float32(np.inf)), np.nextafter(base, np.float32(0))):
            b = (rng.standard_normal(32) * float(base) / 4).astype(np.float32)
            b[rng.integers(32)] = a
            blocks.append(b)
    blocks.append(np.zeros(32, np.float32))
    return np.stack(blocks).astype(np.float32)


def main():
    sys.path.insert(0, REF_GOLDEN)
    import golden as G  # the reference's bit primitives (definitions only)

    rng = np.random.default_rng(4104)
    x = inputs(rng)
    codes = np.zeros(x.shape, np.uint8)
    scales = np.zeros(x.shape[0], np.uint8)
    for bi, blk in enumerate(x):
        amax = np.float32(0.0)
        for v in blk:
            av = np.float32(abs(v))
            if av > amax:
                amax = av
        if float(amax) == 0.0:
            continue
        e = G.block_exp(G.f32_bits(amax))
        scales[bi] = min(max(e + 127, 0), 254)
        p2 = np.float32(G.pow2_neg_e(e))
        for j in range(32):
            codes[bi, j] = G.fp8_code_rshift(np.float32(np.float32(blk[j]) * p2))
    out = os.path.join(HERE, "r4_blocks.npz")
    np.savez_compressed(out, x=x, codes=codes, scales=scales)
    print(out, x.shape[0], "blocks")


if __name__ == "__main__":
    main()
