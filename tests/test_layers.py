"""The layer module on the CPU (no GPU): configuration, errors, naming, the finite guard, and
Linear / Conv2d forward and backward on CPU tensors against the oracle, bit for bit. The GPU
numerics are in test_gpu_linear.py and test_gpu_conv.py."""
import numpy as np
import pytest
import torch

import bit_reproducible_training_amd as rg
from oracle import oracle as O


def bits(t):
    return np.ascontiguousarray(t.detach().numpy() if hasattr(t, "detach") else t, np.float32).view(np.uint32)


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


@pytest.mark.parametrize("S", [1, 2, 3])
def test_linear_on_cpu_matches_oracle(S):
    """Forward, dX, dW and db of a CPU Linear layer equal the definitions computed by the
    oracle: y = fl(gemm(x, W^T) + b), dX = gemm(dY, W), dW = gemm(dY^T, x), db = exact column
    sum of dY."""
    torch.manual_seed(S)
    m, n_in, n_out = 13, 29, 7
    lin = rg.Linear(n_in, n_out)
    x = torch.randn(m, n_in, requires_grad=True)
    dy = torch.randn(m, n_out)
    rg.set_slices(S)
    try:
        y = lin(x)
        y.backward(dy)
    finally:
        rg.set_slices(3)
    xn, wn, bn, dyn = (t.detach().numpy() for t in (x, lin.weight, lin.bias, dy))
    prod = O.cpu_gemm(xn, wn, m, n_out, n_in, 0, 1, S)
    assert np.array_equal(bits(y), bits(prod + bn[None, :]))
    assert np.array_equal(bits(x.grad), bits(O.cpu_gemm(dyn, wn, m, n_in, n_out, 0, 0, S)))
    assert np.array_equal(bits(lin.weight.grad), bits(O.cpu_gemm(dyn, xn, n_out, n_in, m, 1, 0, S)))
    assert np.array_equal(bits(lin.bias.grad), bits(O.exact_sum(dyn, m, n_out, 1)))


def test_linear_leading_dimensions_and_slices_fixed_at_forward():
    """[B, T, in] input is the GEMM over B*T rows; backward uses the S of its forward pass."""
    torch.manual_seed(0)
    lin = rg.Linear(6, 5, bias=False)
    x = torch.randn(2, 3, 6, requires_grad=True)
    rg.set_slices(1)
    try:
        y = lin(x)
    finally:
        rg.set_slices(3)
    dy = torch.randn(2, 3, 5)
    y.backward(dy)                              # S = 1 still, although S = 3 is now set
    xn, wn, dyn = x.detach().numpy().reshape(6, 6), lin.weight.detach().numpy(), dy.numpy().reshape(6, 5)
    assert y.shape == (2, 3, 5)
    assert np.array_equal(bits(y).reshape(6, 5), bits(O.cpu_gemm(xn, wn, 6, 5, 6, 0, 1, 1)))
    assert np.array_equal(bits(x.grad).reshape(6, 6), bits(O.cpu_gemm(dyn, wn, 6, 6, 5, 0, 0, 1)))
    assert np.array_equal(bits(lin.weight.grad), bits(O.cpu_gemm(dyn, xn, 5, 6, 6, 1, 0, 1)))


def test_conv2d_on_cpu_matches_oracle():
    torch.manual_seed(1)
    conv = rg.Conv2d(3, 4, (3, 2), stride=(2, 1), padding=(1, 0))
    x = torch.randn(2, 3, 9, 7, requires_grad=True)
    y = conv(x)
    dy = torch.randn_like(y) * 1e-3
    y.backward(dy)
    shape = (2, 3, 9, 7, 4, 3, 2, 2, 1, 1, 0)
    xn, wn, bn, dyn = (t.detach().numpy() for t in (x, conv.weight, conv.bias, dy))
    assert np.array_equal(bits(y), bits(O.conv2d(xn, wn, shape) + bn[None, :, None, None]))
    assert np.array_equal(bits(x.grad), bits(O.conv2d_grad_input(dyn, wn, shape)))
    assert np.array_equal(bits(conv.weight.grad), bits(O.conv2d_grad_weight(dyn, xn, shape)))
    n, f, oh, ow = dyn.shape
    assert np.array_equal(bits(conv.bias.grad), bits(O.exact_sum(dyn, n, f, oh * ow)))


def test_conv2d_padding_forms():
    assert rg.Conv2d(2, 2, 3, padding="same")._zero_padding() == (1, 1)
    assert rg.Conv2d(2, 2, 3, padding="valid")._zero_padding() == (0, 0)
    for bad in (dict(groups=2), dict(dilation=2), dict(padding_mode="reflect", padding=1)):
        with pytest.raises(NotImplementedError):
            rg.Conv2d(2, 2, 3, **bad)(torch.randn(1, 2, 5, 5))
    with pytest.raises(NotImplementedError):
        rg.Conv2d(2, 2, 2, padding="same")(torch.randn(1, 2, 5, 5))


def test_finite_guard_on_cpu_names_first_operation():
    g = rg.FiniteGuard()
    x = torch.ones(5)
    g.scan(x, "a input")
    g.check()
    x[3] = float("nan")
    g.scan(x, "b weight")
    g.scan(x, "a input")                        # first used earlier, so reported first
    with pytest.raises(FloatingPointError, match="a input at step 4"):
        g.check(4)
    assert g.first_offender() == "a input"
    g.reset()
    g.check()
    lin = rg.Linear(3, 2)
    lin.repro_name = "cpu probe"
    rg.guard().reset()
    lin(torch.tensor([[1.0, float("inf"), 0.0]]))
    with pytest.raises(FloatingPointError, match="cpu probe input"):
        rg.guard().check()
    rg.guard().reset()
