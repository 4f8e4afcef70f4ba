"""INTEGRATION.md's C example, compiled as C99 against include/mxfa.h and linked with
libmxfa.so, then run: the plan and argument-validation calls need no GPU."""
import os
import re
import shutil
import subprocess

import pytest

import mxfa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def example_source():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```c\n(.*?)```", text, flags=re.S)
    return next(b for b in blocks if "int main(void)" in b)


@pytest.mark.skipif(shutil.which("cc") is None, reason="no C compiler")
def test_integration_c_example_compiles_and_runs(tmp_path):
    src = tmp_path / "example.c"
    src.write_text(example_source())
    exe = tmp_path / "example"
    libdir = os.path.dirname(mxfa.LIB_PATH)
    subprocess.run(["cc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), str(src), "-o",
                    str(exe), "-L", libdir, "-lmxfa", f"-Wl,-rpath,{libdir}"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert f"prefill workspace {2 * 8 * 4096 * 128 * 2} bytes" in out.stdout
    assert "argument checks ok" in out.stdout
    assert "invalid argument" in out.stderr          # run_prefill reported the NULL operands
