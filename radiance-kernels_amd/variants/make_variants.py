"""Build the prefill variants measured against the shipped kernel (not part of the library).

Each variant is the shipped kernel source with one change, applied by exact text
replacement to a copy of csrc/ under variants/_build/<name>/ and compiled with the
library's own flags into variants/mxfa_kernels_<name>.hsaco.  Point MXFA_HSACO at one
to run it through libmxfa (bench.py --profile c3 and rocprofv3, for instance).
(Occupancy variants need no build: MXFA_PREFILL_LDS_PAD=<bytes> adds dynamic LDS to the
shipped code object's prefill launches.)
  q_e4m3  Q held as its E4M3 codes and E8M0 scales (20 registers instead of 32) and
          widened to bf16 per score-MFMA pair with v_cvt_scalef32_pk_bf16_fp8 (an empty asm
          statement keeps the compiler from hoisting the loop-invariant conversion out of the
          key loop, which would undo the variant)
  four_wg four workgroups (four waves per SIMD) per CU: launch bounds of four, one K stage at
          D = 128 (33 KB of LDS), so the compiler has 128 registers per lane
Usage: python make_variants.py [name ...]   (default: all)"""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "csrc")
HIPCC = os.path.join(os.environ.get("ROCM", "/opt/rocm"), "bin", "hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]

Q_E4M3 = [
    ("k_prefill.hip", '''  v4i qb[D / 16];
  load_q<D>(qb, a.q + (bh * a.Sq + qi) * D, a.qs + (bh * a.Sq + qi) * (D / 32), qvalid, h);
''', '''  v2i qw[D / 16];
  float qsc[D / 32];
  {
    const uint8_t* qrow = a.q + (bh * a.Sq + qi) * D;
    const uint8_t* qsrow = a.qs + (bh * a.Sq + qi) * (D / 32);
#pragma unroll
    for (int kk = 0; kk < D / 16; kk++)
      qw[kk] = qvalid ? *reinterpret_cast<const v2i*>(qrow + 16 * kk + 8 * h) : (v2i){0, 0};
#pragma unroll
    for (int g = 0; g < D / 32; g++) qsc[g] = qvalid ? e8m0_as_float(qsrow[g]) : 0.0f;
  }
'''),
    ("k_prefill.hip", '''    p3_qk<D>(sc, qb, kb_cur, SOFTCAP ? fresh_lane() : lane);''',
     '''    p3_qk_e8<D>(sc, qw, qsc, kb_cur, SOFTCAP ? fresh_lane() : lane);'''),
    ("k_prefill.hip", '''// ---- Workspace-free form (mxfa_prefill)''', '''template <int D>
__device__ __forceinline__ void p3_qk_e8(v16f (&s)[BN / 32], const v2i* qw, const float* qsc, const uint8_t* kb,
                                         int lane) {
  const int r = lane & 31, h = lane >> 5;
  const uint8_t* kbase = kb + (r / 16) * (32 * D) + h * 256 + (r % 16) * 16;
#pragma unroll
  for (int t = 0; t < BN / 32; t++) s[t] = (v16f){};
#pragma unroll
  for (int kk = 0; kk < D / 16; kk++) {
    v2i w = qw[kk];
    __asm__ volatile("" : "+v"(w));
    const v4i q = fp8x8_to_bf16x8((uint32_t)w[0], (uint32_t)w[1], qsc[kk / 2]);
#pragma unroll
    for (int t = 0; t < BN / 32; t++)
      s[t] = mfma_bf16(*reinterpret_cast<const v4i*>(kbase + t * 2 * (32 * D) + kk * 512), q, s[t]);
  }
}

// ---- Workspace-free form (mxfa_prefill)'''),
]

FOUR_WG = [
    ("k_prefill.hip", "template <int D> constexpr bool p3_one_k_stage() { return D == 256; }",
     "template <int D> constexpr bool p3_one_k_stage() { return D >= 128; }"),
    ("k_prefill.hip", "__launch_bounds__(64 * P3Waves<D>::N, p3_one_k_stage<D>() ? 2 : 3) NAME(FaArgs a)",
     "__launch_bounds__(64 * P3Waves<D>::N, D == 256 ? 2 : 4) NAME(FaArgs a)"),
]

VARIANTS = {"q_e4m3": Q_E4M3, "four_wg": FOUR_WG}


def apply(name, src):
    """Copy csrc/ to src and apply the variant's replacements there."""
    shutil.rmtree(src, ignore_errors=True)
    shutil.copytree(CSRC, src)
    for fname, old, new in VARIANTS[name]:
        path = os.path.join(src, fname)
        text = open(path).read()
        if text.count(old) != 1:
            raise SystemExit(f"{name}: the text to replace in {fname} is not found exactly once")
        open(path, "w").write(text.replace(old, new))


def build(name):
    src = os.path.join(HERE, "_build", name)
    apply(name, src)
    out = os.path.join(HERE, f"mxfa_kernels_{name}.hsaco")
    subprocess.run([HIPCC, "--genco", *FLAGS, f"-I{src}", "-o", out, os.path.join(src, "mxfa_kernels.hip")],
                   check=True)
    print(out)


if __name__ == "__main__":
    for n in sys.argv[1:] or VARIANTS:
        build(n)
