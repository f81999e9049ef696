"""GPU parity of the reproducible convolution (include/repro_conv.h) and the Conv2d layer.

Mirrors repro_conv_cuda/test_repro_conv.cu (GPU equals the CPU definition bit for bit for the
forward pass and both gradients at S = 1, 2, 3, several strides and paddings) and the
reference suite's LeNet convolution hashes (gpt2_ops_suite/results/mac/cpu.txt:35-39).
"""
import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from gpu_util import note, to_dev
from oracle import oracle as O
from test_conv import SHAPES, suite_conv_cases

pytestmark = pytest.mark.gpu


def _t(torch, a, shape):
    return to_dev(torch, a).reshape(shape)


def _run(torch, kind, a, b, shape, S):
    N, C, H, W, F, KH, KW, SY, SX, PY, PX = shape
    OH, OW = O.conv_out_hw(shape)
    if kind == "fwd":
        out = rg.conv2d(_t(torch, a, (N, C, H, W)), _t(torch, b, (F, C, KH, KW)), SY, SX, PY, PX, S)
    elif kind == "dW":
        out = rg.conv2d_grad_weight(_t(torch, a, (N, F, OH, OW)), _t(torch, b, (N, C, H, W)), KH,
                                    KW, SY, SX, PY, PX, S)
    else:
        out = rg.conv2d_grad_input(_t(torch, a, (N, F, OH, OW)), _t(torch, b, (F, C, KH, KW)),
                                   (N, C, H, W), SY, SX, PY, PX, S)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _oracle(kind, a, b, shape, S):
    return {"fwd": O.conv2d, "dW": O.conv2d_grad_weight, "dX": O.conv2d_grad_input}[kind](
        a, b, shape, S)


def test_suite_conv_hashes_gpu(torch_gpu):
    for case in suite_conv_cases():
        note("conv suite", case["name"])
        out = _run(torch_gpu, case["kind"], *case["inputs"], case["shape"], 3)
        assert "%016x" % O.fnv1a64(out) == case["golden"]["out_hash"], case["name"]


@pytest.mark.parametrize("S", [1, 2, 3])
def test_conv_matches_oracle(torch_gpu, S):
    torch = torch_gpu
    shapes = SHAPES + [(16, 3, 32, 32, 8, 3, 3, 1, 1, 1, 1), (4, 8, 20, 20, 12, 5, 5, 2, 2, 2, 2)]
    for shape in shapes:
        rng = np.random.default_rng(sum(shape) * 3 + S)
        N, C, H, W, F, KH, KW = shape[:7]
        OH, OW = O.conv_out_hw(shape)
        x = rng.standard_normal(N * C * H * W).astype(np.float32)
        w = (rng.standard_normal(F * C * KH * KW) * 0.1).astype(np.float32)
        # dY with a different magnitude per image exercises the per-image scales.
        dy = (rng.standard_normal((N, F * OH * OW)) *
              (np.float32(2.0) ** rng.integers(-30, 30, (N, 1)))).astype(np.float32).reshape(-1)
        for kind, a, b in (("fwd", x, w), ("dW", dy, x), ("dX", dy, w)):
            note("conv", kind, shape, "S=%d" % S)
            got = _run(torch, kind, a, b, shape, S)
            want = _oracle(kind, a, b, shape, S)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (kind, shape, S)


def test_conv_wide_dynamic_range(torch_gpu):
    """Inputs spanning 2^-60 .. 2^60 with zeros: scales, clamps and roundings at the edges."""
    torch = torch_gpu
    shape = (6, 4, 11, 11, 5, 3, 3, 2, 1, 1, 2)
    N, C, H, W, F, KH, KW = shape[:7]
    OH, OW = O.conv_out_hw(shape)
    rng = np.random.default_rng(99)

    def wide(n):
        v = rng.standard_normal(n) * 2.0 ** rng.integers(-60, 60, n)
        v[rng.random(n) < 0.05] = 0.0
        return v.astype(np.float32)

    x, w, dy = wide(N * C * H * W), wide(F * C * KH * KW), wide(N * F * OH * OW)
    for kind, a, b in (("fwd", x, w), ("dW", dy, x), ("dX", dy, w)):
        note("conv wide", kind)
        got = _run(torch, kind, a, b, shape, 3)
        want = _oracle(kind, a, b, shape, 3)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), kind


def test_conv2d_layer_forward_backward(torch_gpu):
    torch = torch_gpu
    shape = (100, 6, 14, 14, 16, 5, 5, 1, 1, 0, 0)   # LeNet conv2, batch 100
    N, C, H, W, F, KH, KW = shape[:7]
    OH, OW = O.conv_out_hw(shape)
    x = O.gen_normal(N * C * H * W, 1.0, 11)
    w = O.gen_normal(F * C * KH * KW, 0.1, 12)
    b = O.gen_normal(F, 0.1, 13)
    dy = O.gen_normal(N * F * OH * OW, 1e-3, 14)
    conv = rg.Conv2d(C, F, KH).cuda()
    with torch.no_grad():
        conv.weight.copy_(torch.from_numpy(w.reshape(F, C, KH, KW)))
        conv.bias.copy_(torch.from_numpy(b))
    xd = _t(torch, x, (N, C, H, W)).requires_grad_(True)
    note("Conv2d layer")
    y = conv(xd)
    y.backward(_t(torch, dy, (N, F, OH, OW)))
    want_y = O.conv2d(x, w, shape, 3) + b.reshape(1, F, 1, 1)
    checks = [(y, want_y, "y"), (xd.grad, O.conv2d_grad_input(dy, w, shape, 3), "dx"),
              (conv.weight.grad, O.conv2d_grad_weight(dy, x, shape, 3), "dw"),
              (conv.bias.grad, O.exact_sum(dy, N, F, OH * OW), "db")]
    for got, want, what in checks:
        g = got.detach().cpu().numpy()
        assert np.array_equal(g.view(np.uint32), want.astype(np.float32).view(np.uint32)), what


def _lenet_like(torch, steps=3):
    """conv(1->6, 5x5, pad 2) -> relu -> conv(6->16, 5x5, stride 2) -> relu -> linear(->10),
    plain SGD; every reduction is reproducible, the rest is elementwise."""
    rg.guard().reset()
    c1, c2 = rg.Conv2d(1, 6, 5, padding=2).cuda(), rg.Conv2d(6, 16, 5, stride=2).cuda()
    fc = rg.Linear(16 * 12 * 12, 10).cuda()
    params = []
    for i, m in enumerate((c1, c2, fc)):
        with torch.no_grad():
            for j, p in enumerate((m.weight, m.bias)):
                p.copy_(torch.from_numpy(O.gen_uniform_pm(p.numel(), np.float32(0.1),
                                                          500 + 10 * i + j)).reshape(p.shape))
                params.append(p)
    rg.name_layers(torch.nn.ModuleDict({"c1": c1, "c2": c2, "fc": fc}))
    for step in range(steps):
        x = _t(torch, O.gen_normal(32 * 28 * 28, 1.0, 900 + step), (32, 1, 28, 28))
        target = _t(torch, O.gen_normal(32 * 10, 1.0, 950 + step), (32, 10))
        h = c1(x)
        h = torch.where(h > 0, h, torch.zeros_like(h))
        h = c2(h)
        h = torch.where(h > 0, h, torch.zeros_like(h))
        out = fc(h.reshape(32, -1))
        out.backward(out.detach() - target)
        with torch.no_grad():
            for p in params:
                p -= 0.01 * p.grad
                p.grad = None
        rg.guard().check(step)
    return O.fnv_chain(*[p.detach().cpu().numpy() for p in params])


def test_conv_training_steps_are_bitwise_repeatable(torch_gpu):
    note("lenet-like run 1")
    first = _lenet_like(torch_gpu)
    note("lenet-like run 2")
    assert _lenet_like(torch_gpu) == first
