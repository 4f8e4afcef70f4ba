"""O of a seeded GQA causal prefill (B=2 Hq=8 Hkv=2 S=1024 D=128, 1% outliers x20) through
libmxfa as the environment configures it (MXFA_HSACO, MXFA_PREFILL_LDS_PAD), saved to OUT.npy;
with --against REF.npy, also compared bit for bit with an earlier run's O (exit status 1 if
they differ).  Needs a GPU.
Usage: python check_variant.py OUT.npy [--against REF.npy]"""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), ".."))
import torch  # noqa: E402

import mxfa  # noqa: E402


def main():
    out_path = sys.argv[1]
    ref = sys.argv[sys.argv.index("--against") + 1] if "--against" in sys.argv else None
    B, Hq, Hkv, S, D = 2, 8, 2, 1024, 128
    x = {n: torch.empty(shape, dtype=torch.float32, device="cuda:0")
         for n, shape in (("Q", (B, Hq, S, D)), ("K", (B, Hkv, S, D)), ("V", (B, Hkv, S, D)))}
    for i, n in enumerate(("Q", "K", "V")):
        mxfa.fill_normal(x[n], 500 + i, 0.01)
    q, qs = mxfa.quantize_rows(x["Q"])
    k, ks = mxfa.quantize_rows(x["K"])
    v, vs = mxfa.quantize_cols(x["V"])
    p = mxfa.make_params(B, Hq, Hkv, S, S, D, causal=True)
    o = mxfa.prefill(p, q, qs, k, ks, v, vs).cpu().numpy()
    np.save(out_path, o)
    if ref is None:
        print(f"saved {out_path}", flush=True)
        return 0
    same = np.array_equal(o, np.load(ref))
    print("bit-identical" if same else f"differs: max {np.abs(o - np.load(ref)).max()}", flush=True)
    return 0 if same else 1


if __name__ == "__main__":
    sys.exit(main())
