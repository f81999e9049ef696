"""The register-only MFMA probe (rg_measure_mfma_int8_rate) in its three operand modes: every
mode reports a finite rate below the dense int8 peak, and zero operands (the least switching
power) run at least as fast as random bytes."""
import math

import pytest

import bit_reproducible_training_amd as rg
from gpu_util import note

pytestmark = pytest.mark.gpu


def test_probe_modes(torch_gpu):
    note("mfma probe modes")
    rand = rg.measure_mfma_int8_rate(True)
    low7 = rg.measure_mfma_int8_rate(low7=True)
    zero = rg.measure_mfma_int8_rate(False)
    for v in (rand, low7, zero):
        assert math.isfinite(v) and 500.0 < v <= 5100.0
    assert zero >= 0.95 * rand
