"""Compiled-code properties the results depend on, checked on the gfx950 assembly of
this library's own sources (no GPU needed)."""
import os
import re
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "bit_reproducible_training_amd", "csrc")


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    from bit_reproducible_training_amd import _build

    out = {}
    for src in ("rg_slice.hip", "rg_contract.hip"):
        path = str(tmp_path_factory.mktemp("asm") / (src + ".s"))
        cmd = [_build.HIPCC] + _build.COMMON_FLAGS + ["--cuda-device-only", "-S",
                                                       os.path.join(CSRC, src), "-o", path]
        subprocess.run(cmd, check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
        with open(path) as f:
            out[src] = f.read()
    return out


def test_f32_denormals_preserved(asm):
    """The slicing kernels round x * 2^n with float multiplications, exact only when f32
    denormals are neither flushed on input nor on output (mode 3)."""
    for src, text in asm.items():
        modes = re.findall(r"\.amdhsa_float_denorm_mode_32 (\d+)", text)
        assert modes and set(modes) == {"3"}, (src, set(modes))


def test_contraction_uses_int8_mfma_without_spills(asm):
    text = asm["rg_contract.hip"]
    assert "v_mfma_i32_32x32x32_i8" in text
    spills = re.findall(r"\.vgpr_spill_count:\s*(\d+)", text)
    assert spills and max(int(s) for s in spills) == 0
