"""The prefill variants that profiles/prefill_c3_variants.txt measures are the shipped kernel
sources with exact text replacements (radiance-kernels_amd/variants/make_variants.py); each
replacement target must still occur exactly once in the current sources, or the recipe no
longer builds what it describes.  CPU only: applies the replacements, compiles nothing."""
import importlib.util
import os

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SCRIPT = os.path.join(HERE, "..", "radiance-kernels_amd", "variants", "make_variants.py")


def _module():
    spec = importlib.util.spec_from_file_location("make_variants", SCRIPT)
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


@pytest.mark.parametrize("name", ["q_e4m3", "four_wg"])
def test_variant_replacements_apply(name, tmp_path):
    m = _module()
    m.apply(name, str(tmp_path / name))
    for fname, _, new in m.VARIANTS[name]:
        assert new in open(tmp_path / name / fname).read()
