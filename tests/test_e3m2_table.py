"""The quantizers' branch-free E3M2 encoder (e3m2_code_tab: bf16 rounding by integer add and
shift, a 14 x 128-entry table filled from the rule itself) against the R1 E3M2 rule
(e3m2_code_bf16(bf16_rne(y))) on all 2^32 float bit patterns.  The header holding both builds
as plain C++, so this compiles it for the host with g++ and runs the comparison on 8 threads
(a few seconds)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "radiance-kernels_amd", "csrc")

DRIVER = r"""
#define __device__
#define __forceinline__ inline
#include "e3m2_rule.h"
#include <atomic>
#include <cstdio>
#include <thread>
#include <vector>
int main() {
  using namespace mxfa;
  uint8_t tab[E3M2_TAB_N];
  e3m2_tab_fill(tab, 0, 1);
  std::atomic<unsigned long long> bad{0};
  std::vector<std::thread> th;
  for (int t = 0; t < 8; t++)
    th.emplace_back([&, t] {
      unsigned long long nb = 0;
      for (unsigned long long u = t; u < (1ull << 32); u += 8) {
        const float y = __builtin_bit_cast(float, (uint32_t)u);
        const uint32_t got = e3m2_code_tab(y, tab), want = e3m2_code_bf16(bf16_rne(y));
        if (got != want && nb++ < 4) std::printf("mismatch %08llx: %u vs %u\n", u, got, want);
      }
      bad += nb;
    });
  for (auto& x : th) x.join();
  std::printf("mismatches %llu\n", bad.load());
  return bad != 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_e3m2_table_encoder_equals_rule_on_every_float(tmp_path):
    src = tmp_path / "e3m2_check.cpp"
    exe = tmp_path / "e3m2_check"
    src.write_text(DRIVER)
    subprocess.run(["g++", "-O2", "-std=c++20", "-pthread", f"-I{CSRC}", str(src), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0 and "mismatches 0" in r.stdout, r.stdout
