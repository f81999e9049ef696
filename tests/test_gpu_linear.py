"""The reproducible Linear layer (autograd) on the GPU.

Forward y = x W^T (+ b), backward dX = dY W, dW = dY^T X through the reproducible GEMM and
db = exact column sum of dY, exactly as repro_torch/repro_torch/layers.py:70-100 defines
them. Checked three ways:
  - the layer reproduces the output hashes the reference recorded for the Linear GEMMs of its
    GPT-2 suite (gpt2_ops_suite/results/mac/cpu.txt:2-16) when fed the suite's inputs;
  - forward, dX, dW, db equal the oracle bit for bit at S = 1, 2, 3 on the LeNet-5 MLP shapes
    (batch 64: 400->120, 120->84, 84->10), bias included;
  - a few SGD steps of a small MLP give identical weights on repeated runs, and the finite
    guard names the first operation that saw a NaN.
"""
import json
import os

import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from gpu_util import note
from oracle import oracle as O

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _suite_ops():
    with open(os.path.join(GOLDEN, "suite_gemm_s3.json")) as f:
        return {op["name"]: op for op in json.load(f)["gemm"]}


def _inputs(op):
    A = O.gen_normal(op["M"] * op["K"], op["sa"], op["seed"])
    B = O.gen_normal(op["K"] * op["N"], op["sb"], op["seed"] + 1)
    assert "%016x" % O.fnv_chain(A, B) == op["in_hash"]
    return A, B


def _hash(t):
    return "%016x" % O.fnv1a64(t.detach().cpu().numpy())


@pytest.mark.parametrize("layer", ["attn_qkv", "attn_proj", "mlp_fc", "mlp_proj", "lm_head"])
def test_linear_reproduces_reference_suite_hashes(torch_gpu, layer):
    torch = torch_gpu
    ops = _suite_ops()
    fwd, dX, dW = ops[layer + ".fwd"], ops[layer + ".dX"], ops[layer + ".dW"]
    n_in, n_out = fwd["K"], fwd["N"]

    # forward: x [tokens][in], W [out][in]  (suite op: A = x, B = W stored N x K)
    x, w = _inputs(fwd)
    lin = rg.Linear(n_in, n_out, bias=False).cuda()
    with torch.no_grad():
        lin.weight.copy_(torch.from_numpy(w.reshape(n_out, n_in)))
    note("linear fwd", layer)
    y = lin(torch.from_numpy(x.reshape(fwd["M"], n_in)).cuda())
    assert _hash(y) == fwd["out_hash"]

    # dX = dY W  (suite op: A = dY [tokens][out], B = W [out][in])
    dy, w = _inputs(dX)
    with torch.no_grad():
        lin.weight.copy_(torch.from_numpy(w.reshape(n_out, n_in)))
    xin = torch.zeros(dX["M"], n_in, device="cuda", requires_grad=True)
    note("linear dX", layer)
    lin(xin).backward(torch.from_numpy(dy.reshape(dX["M"], n_out)).cuda())
    assert _hash(xin.grad) == dX["out_hash"]

    # dW = dY^T X  (suite op: A = dY stored [tokens][out], B = X [tokens][in])
    dy, x = _inputs(dW)
    lin.weight.grad = None
    note("linear dW", layer)
    lin(torch.from_numpy(x.reshape(dW["K"], n_in)).cuda()).backward(
        torch.from_numpy(dy.reshape(dW["K"], n_out)).cuda())
    assert _hash(lin.weight.grad) == dW["out_hash"]


@pytest.mark.parametrize("S", [1, 2, 3])
def test_linear_forward_backward_match_oracle(torch_gpu, S):
    torch = torch_gpu
    rg.set_slices(S)
    try:
        batch = 64
        for i, (n_in, n_out) in enumerate([(400, 120), (120, 84), (84, 10)]):
            bound = np.float32(1.0 / np.sqrt(n_in))
            w = O.gen_uniform_pm(n_out * n_in, bound, 2024 + i).reshape(n_out, n_in)
            b = O.gen_uniform_pm(n_out, bound, 3024 + i)
            x = O.gen_normal(batch * n_in, 1.0, 4024 + i).reshape(batch, n_in)
            dy = O.gen_normal(batch * n_out, 1.0, 5024 + i).reshape(batch, n_out)
            lin = rg.Linear(n_in, n_out).cuda()
            with torch.no_grad():
                lin.weight.copy_(torch.from_numpy(w))
                lin.bias.copy_(torch.from_numpy(b))
            xd = torch.from_numpy(x).cuda().requires_grad_(True)
            note("linear S=%d" % S, n_in, n_out)
            y = lin(xd)
            y.backward(torch.from_numpy(dy).cuda())
            want_y = O.cpu_gemm(x, w, batch, n_out, n_in, False, True, S) + b[None, :]
            want_dx = O.cpu_gemm(dy, w, batch, n_in, n_out, False, False, S)
            want_dw = O.cpu_gemm(dy, x, n_out, n_in, batch, True, False, S)
            want_db = O.exact_sum(dy, batch, n_out, 1)
            for got, want, what in [(y, want_y, "y"), (xd.grad, want_dx, "dx"),
                                    (lin.weight.grad, want_dw, "dw"), (lin.bias.grad, want_db, "db")]:
                g = got.detach().cpu().numpy().astype(np.float32)
                assert np.array_equal(g.view(np.uint32), want.astype(np.float32).view(np.uint32)), \
                    (S, n_in, n_out, what)
    finally:
        rg.set_slices(3)


def _train(torch, steps=4):
    """A few plain SGD steps of a 3-layer MLP; the update and activations are elementwise
    (correctly rounded, order-free), every reduction is a reproducible GEMM or exact sum."""
    rg.guard().reset()
    dims = [(400, 120), (120, 84), (84, 10)]
    layers = []
    for i, (n_in, n_out) in enumerate(dims):
        lin = rg.Linear(n_in, n_out).cuda()
        bound = np.float32(1.0 / np.sqrt(n_in))
        with torch.no_grad():
            lin.weight.copy_(torch.from_numpy(
                O.gen_uniform_pm(n_out * n_in, bound, 77 + i).reshape(n_out, n_in)))
            lin.bias.copy_(torch.from_numpy(O.gen_uniform_pm(n_out, bound, 88 + i)))
        layers.append(lin)
    rg.name_layers(torch.nn.Sequential(*layers))
    for step in range(steps):
        x = torch.from_numpy(O.gen_normal(64 * 400, 1.0, 1000 + step).reshape(64, 400)).cuda()
        target = torch.from_numpy(O.gen_normal(64 * 10, 1.0, 2000 + step).reshape(64, 10)).cuda()
        h = x
        for j, lin in enumerate(layers):
            h = lin(h)
            if j + 1 < len(layers):
                h = torch.where(h > 0, h, torch.zeros_like(h))
        (h).backward(h.detach() - target)      # gradient of 0.5 * |h - target|^2
        with torch.no_grad():
            for lin in layers:
                for p in (lin.weight, lin.bias):
                    p -= 0.01 * p.grad
                    p.grad = None
        rg.guard().check(step)
    return [O.fnv_chain(*[p.detach().cpu().numpy() for lin in layers
                          for p in (lin.weight, lin.bias)])]


def test_training_steps_are_bitwise_repeatable(torch_gpu):
    torch = torch_gpu
    note("mlp training run 1")
    first = _train(torch)
    note("mlp training run 2")
    assert _train(torch) == first


def test_finite_guard_names_first_nonfinite_operation(torch_gpu):
    torch = torch_gpu
    g = rg.guard()
    lin = rg.Linear(16, 8).cuda()
    lin.repro_name = "probe"
    x = torch.randn(4, 16, device="cuda")
    note("guard clean")
    lin(x)
    g.check()                                   # nothing non-finite so far
    x[2, 5] = float("nan")
    note("guard nan input")
    lin(x)
    with pytest.raises(FloatingPointError, match="probe input at step 7"):
        g.check(7)
    g.reset()
    g.check()
    with torch.no_grad():
        lin.weight[0, 0] = float("inf")
    lin(torch.randn(4, 16, device="cuda"))
    with pytest.raises(FloatingPointError, match="probe weight"):
        g.check()
    g.reset()


@pytest.mark.parametrize("S", [1, 3])
def test_linear_cpu_and_gpu_give_identical_bits(torch_gpu, S):
    """The same Linear step on CPU tensors (the CPU implementation in the compiled binding) and
    on GPU tensors (the MI355X kernels): forward, dX, dW and db bit for bit."""
    torch = torch_gpu
    torch.manual_seed(10 + S)
    m, n_in, n_out = 192, 400, 120
    cpu = rg.Linear(n_in, n_out)
    gpu = rg.Linear(n_in, n_out).cuda()
    with torch.no_grad():
        gpu.weight.copy_(cpu.weight)
        gpu.bias.copy_(cpu.bias)
    x = torch.randn(m, n_in)
    dy = torch.randn(m, n_out)
    rg.set_slices(S)
    try:
        xc = x.clone().requires_grad_(True)
        yc = cpu(xc)
        yc.backward(dy)
        note("linear cpu vs gpu", S)
        xg = x.cuda().requires_grad_(True)
        yg = gpu(xg)
        yg.backward(dy.cuda())
        torch.cuda.synchronize()
    finally:
        rg.set_slices(3)
    for a, b in ((yc, yg), (xc.grad, xg.grad), (cpu.weight.grad, gpu.weight.grad),
                 (cpu.bias.grad, gpu.bias.grad)):
        assert torch.equal(a.detach().view(torch.int32), b.detach().cpu().view(torch.int32))
