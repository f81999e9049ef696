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
    # The last: windows of 4680 values, too long for the one-pass slicing, so the forward
    # pass packs the im2col matrix instead of gathering it.
    shapes = SHAPES + [(16, 3, 32, 32, 8, 3, 3, 1, 1, 1, 1), (4, 8, 20, 20, 12, 5, 5, 2, 2, 2, 2),
                       (1, 520, 5, 5, 3, 3, 3, 1, 1, 1, 1)]
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


RC = rg.repro_conv
PASSES = {"fwd": RC.FORWARD, "dW": RC.GRAD_WEIGHT, "dX": RC.GRAD_INPUT}


def _run_algo(torch, kind, a, b, shape, S, algo):
    """One pass through the diagnostic hook with its algorithm forced."""
    N, C, H, W, F, KH, KW = shape[:7]
    OH, OW = O.conv_out_hw(shape)
    g = RC.ConvShape(*shape)
    out_shape = {"fwd": (N, F, OH, OW), "dW": (F, C, KH, KW), "dX": (N, C, H, W)}[kind]
    out = torch.full(out_shape, float("nan"), dtype=torch.float32, device="cuda")
    nbytes = RC.conv2d_algo_workspace(PASSES[kind], g, S, algo)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
    da, db = to_dev(torch, a), to_dev(torch, b)
    code = RC.repro_conv2d_algo_ws(PASSES[kind], da.data_ptr(), db.data_ptr(), out.data_ptr(), g,
                                   S, algo, ws.data_ptr(), ws.numel(),
                                   torch.cuda.current_stream().cuda_stream)
    if code != 0:
        raise rg.ReproGemmError(code, "conv algo")
    torch.cuda.synchronize()
    return out.cpu().numpy()


LENET = [(100, 1, 28, 28, 6, 5, 5, 1, 1, 2, 2), (100, 6, 14, 14, 16, 5, 5, 1, 1, 0, 0)]
# Both algorithms on shapes with strides larger than, equal to and smaller than the kernel,
# asymmetric padding, 1x1 kernels, planes smaller and larger than a block of 256 pixels, more
# filters than one pass of accumulators, and the direct kernels' limits: 2048 products per
# input-gradient sum (128 filters x 4x4) with 6144 staged dY values, 2048 per window and 4096
# (padded) weights forward.
DIRECT_SHAPES = SHAPES + [
    (16, 3, 32, 32, 8, 3, 3, 1, 1, 1, 1), (4, 8, 20, 20, 12, 5, 5, 2, 2, 2, 2),
    (2, 3, 17, 19, 9, 3, 5, 4, 3, 0, 2), (3, 2, 40, 13, 17, 1, 1, 1, 1, 0, 0),
    (1, 2, 3, 5, 128, 4, 4, 1, 1, 3, 3), (1, 128, 4, 4, 2, 4, 4, 1, 1, 1, 1),
] + LENET


@pytest.mark.parametrize("S", [1, 2, 3])
def test_direct_and_gemm_algorithms_match_oracle(torch_gpu, S):
    """Forward and input gradient by the direct kernels and by the GEMM pipeline, against the
    oracle bit for bit; the weight gradient (GEMM only) reports not supported for DIRECT."""
    torch = torch_gpu
    for shape in DIRECT_SHAPES:
        if S != 3 and shape in LENET:
            continue
        rng = np.random.default_rng(sum(shape) * 5 + S)
        N, C, H, W, F, KH, KW = shape[:7]
        OH, OW = O.conv_out_hw(shape)
        x = (rng.standard_normal(N * C * H * W) *
             (np.float32(2.0) ** rng.integers(-20, 20, N * C * H * W))).astype(np.float32)
        x[rng.random(x.size) < 0.1] = 0.0
        w = (rng.standard_normal(F * C * KH * KW) * 0.1).astype(np.float32)
        dy = (rng.standard_normal((N, F * OH * OW)) *
              (np.float32(2.0) ** rng.integers(-30, 30, (N, 1)))).astype(np.float32).reshape(-1)
        for kind, a, b in (("fwd", x, w), ("dX", dy, w)):
            want = _oracle(kind, a, b, shape, S).view(np.uint32)
            for algo in (RC.ALGO_DIRECT, RC.ALGO_GEMM, RC.ALGO_AUTO):
                note("conv algo", kind, shape, "S=%d algo=%d" % (S, algo))
                got = _run_algo(torch, kind, a, b, shape, S, algo)
                assert np.array_equal(got.view(np.uint32), want), (kind, shape, S, algo)
        g = RC.ConvShape(*shape)
        with pytest.raises(rg.ReproGemmError):
            RC.conv2d_algo_workspace(RC.GRAD_WEIGHT, g, S, RC.ALGO_DIRECT)


def test_gemm_pipeline_beyond_65535_images(torch_gpu):
    """More images than a grid's y dimension holds: the [N][F][P] <-> [N*P][F] reorders fall
    back from the tiled transposes to their element-wise kernels (GEMM algorithm forced)."""
    torch = torch_gpu
    shape = (65537, 2, 3, 2, 3, 2, 1, 1, 1, 0, 0)
    N, C, H, W, F, KH, KW = shape[:7]
    OH, OW = O.conv_out_hw(shape)
    rng = np.random.default_rng(65537)
    x = rng.standard_normal(N * C * H * W).astype(np.float32)
    w = (rng.standard_normal(F * C * KH * KW) * 0.1).astype(np.float32)
    dy = (rng.standard_normal((N, F * OH * OW)) *
          (np.float32(2.0) ** rng.integers(-20, 20, (N, 1)))).astype(np.float32).reshape(-1)
    for kind, a, b in (("fwd", x, w), ("dW", dy, x), ("dX", dy, w)):
        note("conv 65537 images", kind)
        got = _run_algo(torch, kind, a, b, shape, 3, RC.ALGO_GEMM)
        want = _oracle(kind, a, b, shape, 3)
        assert np.array_equal(got.view(np.uint32).reshape(-1), want.view(np.uint32).reshape(-1)), kind


def test_direct_sums_at_their_exactness_limit(torch_gpu):
    """Every value 127 = 127 * 2^0, which its scale (2^0) maps to the largest fixed-point
    value X = 127 * 2^14: the central pixel's input-gradient sum has 2048 products of
    (127 * 2^14)^2 = 2^41.98 each, a forward window sum 2048, so the binary64 sums reach
    +-2048 * (127 * 2^14)^2, just below 2^53, and must stay exact."""
    torch = torch_gpu
    for kind, shape in (("dX", (1, 1, 3, 3, 128, 4, 4, 1, 1, 3, 3)),
                        ("fwd", (2, 128, 4, 4, 2, 4, 4, 1, 1, 0, 0))):
        N, C, H, W, F, KH, KW = shape[:7]
        OH, OW = O.conv_out_hw(shape)
        x = np.full(N * C * H * W, 127.0, np.float32)
        dy = np.full(N * F * OH * OW, 127.0, np.float32)
        for sign in (1.0, -1.0):
            w = np.full(F * C * KH * KW, sign * 127.0, np.float32)
            a = x if kind == "fwd" else dy
            want = _oracle(kind, a, w, shape, 3)
            assert np.abs(want).max() == np.float32(2048 * 127.0 ** 2)
            for algo in (RC.ALGO_DIRECT, RC.ALGO_GEMM):
                note("conv limit", kind, shape, sign, "algo=%d" % algo)
                got = _run_algo(torch, kind, a, w, shape, 3, algo)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (kind, algo)


def test_conv_algorithm_choice(torch_gpu):
    """Small filters take the direct kernels (LeNet conv1 both passes, conv2's input gradient;
    conv2's forward, 1200 multiply-adds per thread, the GEMM pipeline), large convolutions and
    the weight gradient the GEMM pipeline; the entry points' workspace is the chosen
    algorithm's."""
    conv1, conv2 = (RC.ConvShape(*s) for s in LENET)
    want = {(0, RC.FORWARD): RC.ALGO_DIRECT, (0, RC.GRAD_INPUT): RC.ALGO_DIRECT,
            (1, RC.FORWARD): RC.ALGO_GEMM, (1, RC.GRAD_INPUT): RC.ALGO_DIRECT}
    for i, g in enumerate((conv1, conv2)):
        for p in (RC.FORWARD, RC.GRAD_INPUT):
            assert RC.conv2d_algo(p, g) == want[(i, p)], (i, p)
        assert RC.conv2d_algo(RC.GRAD_WEIGHT, g) == RC.ALGO_GEMM
    assert rg.conv2d_workspace(conv1) == RC.conv2d_algo_workspace(RC.FORWARD, conv1, 3, RC.ALGO_DIRECT)
    assert rg.conv2d_workspace(conv2) == RC.conv2d_algo_workspace(RC.FORWARD, conv2, 3, RC.ALGO_GEMM)
    big = RC.ConvShape(64, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1)
    for p in (RC.FORWARD, RC.GRAD_WEIGHT, RC.GRAD_INPUT):
        assert RC.conv2d_algo(p, big) == RC.ALGO_GEMM
    assert rg.conv2d_grad_input_workspace(big) == RC.conv2d_algo_workspace(
        RC.GRAD_INPUT, big, 3, RC.ALGO_GEMM)
    # Beyond the direct kernels' limits: more dY rows than the staging holds (input gradient),
    # a window of more than 2048 values (forward).
    with pytest.raises(rg.ReproGemmError):
        RC.conv2d_algo_workspace(RC.GRAD_INPUT, RC.ConvShape(1, 2, 12, 12, 128, 4, 4, 1, 1, 3, 3),
                                 3, RC.ALGO_DIRECT)
    with pytest.raises(rg.ReproGemmError):
        RC.conv2d_algo_workspace(RC.FORWARD, RC.ConvShape(1, 129, 6, 6, 1, 4, 4), 3, RC.ALGO_DIRECT)


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


@pytest.mark.parametrize("S", [1, 3])
def test_conv_equals_gpu_gemm_on_im2col(torch_gpu, S):
    """The reference's consumer cross-check (test_repro_conv.cu:84-112) on the GPU: the
    convolution's forward pass equals the GEMM of the im2col matrix with the filters (W^T), and
    its weight gradient the GEMM of dY^T with the im2col matrix, bit for bit, both computed on
    the GPU (whichever algorithm each entry point picks)."""
    from test_conv import im2col

    torch = torch_gpu
    for shape in SHAPES + [(16, 3, 32, 32, 8, 3, 3, 1, 1, 1, 1), (100, 6, 14, 14, 16, 5, 5, 1, 1, 0, 0)]:
        rng = np.random.default_rng(sum(shape) * 5 + S)
        N, C, H, W, F, KH, KW = shape[:7]
        OH, OW = O.conv_out_hw(shape)
        x = rng.standard_normal(N * C * H * W).astype(np.float32)
        w = (rng.standard_normal(F * C * KH * KW) * 0.1).astype(np.float32)
        dy = (rng.standard_normal(N * F * OH * OW) * 1e-3).astype(np.float32)
        cols = im2col(x, shape)
        Wn, K = cols.shape
        note("conv vs gemm", shape, "S=%d" % S)
        y = _run(torch, "fwd", x, w, shape, S)
        g = rg.gemm(to_dev(torch, cols).reshape(Wn, K), to_dev(torch, w).reshape(F, K), Wn, F, K,
                    False, True, S)
        torch.cuda.synchronize()
        want = np.ascontiguousarray(g.cpu().numpy().reshape(N, OH, OW, F).transpose(0, 3, 1, 2))
        assert np.array_equal(y.view(np.uint32).ravel(), want.view(np.uint32).ravel()), shape
        dw = _run(torch, "dW", dy, x, shape, S)
        D = np.ascontiguousarray(dy.reshape(N, F, OH * OW).transpose(0, 2, 1).reshape(Wn, F))
        g = rg.gemm(to_dev(torch, D).reshape(Wn, F), to_dev(torch, cols).reshape(Wn, K), F, K, Wn,
                    True, False, S)
        torch.cuda.synchronize()
        assert np.array_equal(dw.view(np.uint32).ravel(), g.cpu().numpy().view(np.uint32).ravel()), shape


@pytest.mark.parametrize("S", [1, 3])
def test_lenet_step_cpu_and_gpu_give_identical_bits(torch_gpu, S):
    """A LeNet-5-shaped network of the reproducible layers (two Conv2d, three Linear; the
    pooling done by stride-2 convolutions so that every reduction is one of the library's), one
    forward and backward pass with a fixed output gradient, on CPU tensors (the CPU half) and on
    GPU tensors (the MI355X kernels): the output, the input gradient and every parameter
    gradient are identical bit for bit. ReLU is exact on both devices."""
    torch = torch_gpu
    torch.manual_seed(40 + S)

    def lenet():
        return torch.nn.Sequential(
            rg.Conv2d(1, 6, 5, padding=2), torch.nn.ReLU(),
            rg.Conv2d(6, 6, 2, stride=2), torch.nn.ReLU(),
            rg.Conv2d(6, 16, 5), torch.nn.ReLU(),
            rg.Conv2d(16, 16, 2, stride=2), torch.nn.ReLU(),
            torch.nn.Flatten(),
            rg.Linear(16 * 5 * 5, 120), torch.nn.ReLU(),
            rg.Linear(120, 84), torch.nn.ReLU(),
            rg.Linear(84, 10))

    cpu = lenet()
    gpu = lenet().cuda()
    gpu.load_state_dict(cpu.state_dict())
    x = torch.randn(64, 1, 28, 28)
    dy = torch.randn(64, 10)
    rg.set_slices(S)
    try:
        xc = x.clone().requires_grad_(True)
        yc = cpu(xc)
        yc.backward(dy)
        note("lenet cpu vs gpu S=%d" % S)
        xg = x.cuda().requires_grad_(True)
        yg = gpu(xg)
        yg.backward(dy.cuda())
        torch.cuda.synchronize()
    finally:
        rg.set_slices(3)
    pairs = [(yc, yg), (xc.grad, xg.grad)]
    pairs += [(a.grad, b.grad) for a, b in zip(cpu.parameters(), gpu.parameters())]
    for i, (a, b) in enumerate(pairs):
        assert torch.equal(a.detach().view(torch.int32), b.detach().cpu().view(torch.int32)), i
