"""Write the golden fixtures under tests/golden/ from the reference's own
lib/golden code, compiled from its sources into oracle/_ref/ by oracle/Makefile.

Run in the container that holds /root/reference:
    make -C oracle && python tests/golden/make_golden.py

Fixtures (data only: inputs and the reference's outputs):
  decode_tables.npz   e4m3 (256 codes), e3m2 (64 codes), e8m0 (255 codes) decoded
                      by fp8_e4m3_decode / fp6_e3m2_decode / fpe8m0_decode
  e3m2_encode.bin     bf16_bits_to_fp6_e3m2_code for all 65536 bf16 patterns
  e4m3_encode.npz     fp8_e4m3_to_code on edge-case and random float inputs
  requant_postpass.npz  mx_golden CLI (MX_OUT_FMT=0): bf16 C, e4m3 codes and
                      e8m0 scales of its block-32 requant post-pass
"""
import ctypes
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402


def e4m3_edge_inputs(rng):
    xs = []
    # just below / at / above every power of two in [-20, 20]
    for e in range(-20, 21):
        base = np.float32(2.0 ** e).view(np.uint32)
        for d in range(-64, 65):
            xs.append(np.uint32(int(base) + d).view(np.float32))
    # ties of the 3-bit mantissa rounding in every binade of the E4M3 range
    for e in range(-7, 10):
        for q in range(8):
            for half in (0x7ffff, 0x80000, 0x80001):
                b = ((e + 127) << 23) | (q << 20) | half
                xs.append(np.uint32(b).view(np.float32))
    xs += [0.0, -0.0, 448.0, 464.0, 479.9, 480.0, 500.0, 511.99, 512.0, 1e30, 2.0 ** -6, 2.0 ** -7,
           float(np.nextafter(np.float32(2.0 ** -6), np.float32(0))), 1e-40, np.inf, -np.inf, np.nan]
    x = np.array(xs, dtype=np.float32)
    x = np.concatenate([x, -x])
    r = rng.standard_normal(50000).astype(np.float32) * np.float32(2.0) ** rng.integers(-10, 10, 50000).astype(np.float32)
    return np.concatenate([x, r]).astype(np.float32)


def run_mx_golden(exe, M, N, K, A, B, SA, SB, out_fmt):
    with tempfile.TemporaryDirectory() as td:
        paths = {}
        for name, arr in (("A", A), ("B", B), ("SA", SA), ("SB", SB)):
            paths[name] = os.path.join(td, name + ".bin")
            arr.astype(np.uint8).tofile(paths[name])
        outp = os.path.join(td, "C.bin")
        env = dict(os.environ)
        env.pop("MX_OUT_FMT", None)
        scp = os.path.join(td, "S.bin")
        if out_fmt is not None:
            env["MX_OUT_FMT"] = str(out_fmt)
            env["MX_SCALES_OUT"] = scp
        subprocess.run([exe, str(M), str(N), str(K), paths["A"], paths["B"], paths["SA"], paths["SB"], outp],
                       check=True, env=env)
        if out_fmt is None:
            return np.fromfile(outp, np.uint16).reshape(M, N)
        return np.fromfile(outp, np.uint8).reshape(M, N), np.fromfile(scp, np.uint8).reshape(M, N // 32)


def random_e4m3_codes(rng, shape, max_exp_field):
    s = rng.integers(0, 2, shape) << 7
    e = rng.integers(0, max_exp_field + 1, shape) << 3
    m = rng.integers(0, 8, shape)
    return (s | e | m).astype(np.uint8)


def main():
    if not O.ref_available():
        raise SystemExit("oracle/_ref not built: run make -C oracle in the container holding /root/reference")
    R = O.ref()
    rng = np.random.default_rng(20261201)
    # decode tables
    e4 = np.array([R.ref_e4m3_decode(c) for c in range(256)], np.float32)
    e3 = np.array([R.ref_e3m2_decode(c) for c in range(64)], np.float32)
    e8 = np.array([R.ref_e8m0_decode(c) for c in range(255)], np.float32)
    np.savez(os.path.join(HERE, "decode_tables.npz"), e4m3=e4, e3m2=e3, e8m0=e8)
    # e3m2 encode over all bf16
    t = np.array([R.ref_e3m2_encode_bf16(b) for b in range(65536)], np.uint8)
    t.tofile(os.path.join(HERE, "e3m2_encode.bin"))
    # e4m3 encode on edge cases
    x = e4m3_edge_inputs(rng)
    codes = np.empty(len(x), np.uint8)
    R.ref_e4m3_encode_array(x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), len(x),
                            codes.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)))
    np.savez(os.path.join(HERE, "e4m3_encode.npz"), x=x, code=codes)
    # mx_golden requant post-pass: C = A*B in the reference's hardware semantics, then requant.
    exe = O.ref_mx_golden_path()
    cases = []
    for (M, N, K, maxe, two_terms) in ((32, 128, 32, 14, False), (32, 128, 32, 13, True), (64, 64, 64, 12, True)):
        A = random_e4m3_codes(rng, (M, K), maxe)
        B = np.zeros((K, N), np.uint8)
        for n in range(N):                    # each column picks 1 or 2 entries of A's row, scaled by 1.0
            B[n % 16, n] = 0x38
            if two_terms:
                B[16 + (n * 7) % 16, n] = 0x38 if n % 3 else 0x40
        SA = rng.integers(110, 145, (K // 32, M)).astype(np.uint8)
        SB = rng.integers(110, 145, (K // 32, N)).astype(np.uint8)
        C = run_mx_golden(exe, M, N, K, A, B, SA, SB, None)
        q, s = run_mx_golden(exe, M, N, K, A, B, SA, SB, 0)
        cases.append((C, q, s))
    np.savez(os.path.join(HERE, "requant_postpass.npz"),
             **{f"C{i}": c[0] for i, c in enumerate(cases)},
             **{f"codes{i}": c[1] for i, c in enumerate(cases)},
             **{f"scales{i}": c[2] for i, c in enumerate(cases)})
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
