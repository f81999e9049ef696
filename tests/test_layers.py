"""Host-side behaviour of the layer module (no GPU): configuration, errors, naming. The
numerics are in test_gpu_linear.py."""
import pytest
import torch

import bit_reproducible_training_amd as rg


def test_slices_setting():
    assert rg.get_slices() == 3                  # layers.py:7 default
    rg.set_slices(2)
    assert rg.get_slices() == 2
    rg.set_slices(3)
    for bad in (0, 4, -1):
        with pytest.raises(ValueError):
            rg.set_slices(bad)


def test_guard_without_scans_is_silent():
    g = rg.FiniteGuard()
    g.check()
    g.check(3)
    g.reset()


def test_name_layers():
    model = torch.nn.Sequential(rg.Linear(4, 3), torch.nn.ReLU(),
                                torch.nn.Sequential(rg.Linear(3, 2)))
    rg.name_layers(model, "net.")
    assert model[0].repro_name == "net.0"
    assert model[2][0].repro_name == "net.2.0"
    assert rg.Linear(2, 2).repro_name == "linear"


def test_linear_on_cpu_tensors_fails_loudly():
    """No CPU path: the layer raises instead of computing something else."""
    lin = rg.Linear(4, 3)
    with pytest.raises(ValueError, match="GPU"):
        lin(torch.randn(2, 4))
