"""The asynchronous entry points inside HIP graphs (torch.cuda.graph capture).

They allocate nothing, synchronise nothing and clear no memory with memset nodes, so a caller
can capture them (serving loops, training steps replayed as graphs). Every replay must give the
bits of the eager call on the same inputs; replays are separated by eager work and device
synchronisations, and one replay runs on new input values written in place.
"""
import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from gpu_util import note
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().numpy().view(np.uint32)


def _capture(torch, fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()                          # warm-up outside the capture (device facts cached)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


@pytest.mark.parametrize("M,N,K,ta,tb,split,tile", [
    (384, 320, 1000, 0, 0, 1, 16), (200, 130, 5000, 1, 0, 3, 16), (256, 64, 4096, 0, 1, 1, 16),
    (1024, 1024, 64, 0, 1, 1, 16),
    (256, 256, 256, 0, 0, 1, 16), (64, 120, 400, 0, 1, 1, 16),    # one-launch small kernel
    (300, 500, 1500, 1, 0, 1, (64, 192)), (500, 300, 700, 0, 1, 2, (192, 64)),   # 12 wavefronts
    (1000, 300, 100, 0, 1, 1, (32, 128)), (2048, 768, 768, 0, 0, 1, (32, 256)),  # band kernel
    (96, 64, 40000, 0, 0, 1, 16), (64, 96, 36000, 1, 0, 2, 16)])  # wide one-read parts of op(B)
def test_gemm_replays_equal_eager(torch_gpu, M, N, K, ta, tb, split, tile):
    torch = torch_gpu
    torch.manual_seed(M + N + K)
    A = torch.randn(M * K, device="cuda")
    B = torch.randn(K * N, device="cuda")
    C = torch.empty(M, N, device="cuda")
    tm, tn = tile if isinstance(tile, tuple) else (tile, tile)
    cfg = rg.Config(trans_a=ta, trans_b=tb, split_k=split, tile_m=tm, tile_n=tn)
    plan = rg.make_plan(M, N, K, cfg)
    if M * N <= 256 * 256 and K <= 512 and tile == 16:
        assert (plan.tile_m, plan.tile_n) == (32, 32)
    if isinstance(tile, tuple):
        assert (plan.tile_m, plan.tile_n) == tile
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")

    def call():
        code = rg.repro_gemm_fp32_ws(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, cfg,
                                     ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
        assert code == 0

    note("graph gemm", M, N, K, ta, tb, split)
    g = _capture(torch, call)
    want = O.cpu_gemm(A.cpu().numpy(), B.cpu().numpy(), M, N, K, ta, tb, 3).view(np.uint32)
    for rep in range(3):
        C.fill_(float("nan"))
        ws.zero_()                     # eager work on the same buffers between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(C), want), rep
    A.copy_(torch.randn(M * K, device="cuda") * 3.0)
    g.replay()
    torch.cuda.synchronize()
    want2 = O.cpu_gemm(A.cpu().numpy(), B.cpu().numpy(), M, N, K, ta, tb, 3).view(np.uint32)
    assert np.array_equal(_bits(C), want2)


def test_batched_and_sum_replays_equal_eager(torch_gpu):
    torch = torch_gpu
    torch.manual_seed(7)
    T, H, D = 256, 4, 64
    q = torch.randn(T, H * D, device="cuda")
    k = torch.randn(T, H * D, device="cuda")
    heads = lambda z: z.view(T, H, D).permute(1, 0, 2)
    scores = torch.empty(H, T, T, device="cuda")
    x = torch.randn(3000, 96, device="cuda")
    bias_grad = torch.empty(96, device="cuda")
    scfg = rg.SumConfig()
    splan = rg.make_sum_plan(3000, 96, 1, scfg)
    sws = torch.empty(max(splan.workspace_bytes, 1), dtype=torch.uint8, device="cuda")

    def call():
        rg.bmm(heads(q), heads(k), False, True, out=scores)
        code = rg.repro_sum_fp32_ws(x.data_ptr(), bias_grad.data_ptr(), 3000, 96, 1, scfg,
                                    sws.data_ptr(), sws.numel(), torch.cuda.current_stream().cuda_stream)
        assert code == 0

    note("graph bmm + sum")
    g = _capture(torch, call)
    qn, kn, xn = q.cpu().numpy(), k.cpu().numpy(), x.cpu().numpy()
    want_s = np.stack([O.cpu_gemm(np.ascontiguousarray(qn[:, h * D:(h + 1) * D]),
                                  np.ascontiguousarray(kn[:, h * D:(h + 1) * D]), T, T, D, 0, 1, 3)
                       for h in range(H)]).view(np.uint32)
    want_b = O.exact_sum(xn, 3000, 96, 1).view(np.uint32)
    for rep in range(3):
        scores.fill_(float("nan"))
        bias_grad.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(scores), want_s), rep
        assert np.array_equal(_bits(bias_grad), want_b), rep


def test_conv_replays_equal_eager(torch_gpu):
    """The three convolution passes of LeNet conv1 in one graph: the forward and the input
    gradient take the direct kernels, the weight gradient the GEMM pipeline (im2col, slicing,
    split-K contraction, parallel reduction)."""
    torch = torch_gpu
    RC = rg.repro_conv
    shape = (100, 1, 28, 28, 6, 5, 5, 1, 1, 2, 2)
    g_ = RC.ConvShape(*shape)
    assert RC.conv2d_algo(RC.FORWARD, g_) == RC.ALGO_DIRECT
    assert RC.conv2d_algo(RC.GRAD_INPUT, g_) == RC.ALGO_DIRECT
    torch.manual_seed(3)
    x = torch.randn(g_.N, g_.C, g_.H, g_.W, device="cuda")
    w = 0.1 * torch.randn(g_.F, g_.C, g_.KH, g_.KW, device="cuda")
    dy = 1e-3 * torch.randn(g_.N, g_.F, g_.OH, g_.OW, device="cuda")
    y, dw, dx = torch.empty_like(dy), torch.empty_like(w), torch.empty_like(x)
    passes = [(rg.repro_conv2d_ws, rg.conv2d_workspace(g_), x, w, y),
              (rg.repro_conv2d_grad_weight_ws, rg.conv2d_grad_weight_workspace(g_), dy, x, dw),
              (rg.repro_conv2d_grad_input_ws, rg.conv2d_grad_input_workspace(g_), dy, w, dx)]
    wss = [torch.empty(max(n, 1), dtype=torch.uint8, device="cuda") for _, n, _, _, _ in passes]

    def call():
        for (fn, _, a, b, o), ws in zip(passes, wss):
            code = fn(a.data_ptr(), b.data_ptr(), o.data_ptr(), g_, 3, ws.data_ptr(), ws.numel(),
                      torch.cuda.current_stream().cuda_stream)
            assert code == 0

    def want():
        xn, wn, dyn = (t.cpu().numpy().reshape(-1) for t in (x, w, dy))
        return [O.conv2d(xn, wn, shape, 3).view(np.uint32),
                O.conv2d_grad_weight(dyn, xn, shape, 3).view(np.uint32),
                O.conv2d_grad_input(dyn, wn, shape, 3).view(np.uint32)]

    note("graph conv passes")
    g = _capture(torch, call)
    w1 = want()
    for rep in range(3):
        for o in (y, dw, dx):
            o.fill_(float("nan"))
        for ws in wss:
            ws.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, exp in zip((y, dw, dx), w1):
            assert np.array_equal(_bits(o).reshape(-1), exp.reshape(-1)), rep
    x.copy_(torch.randn(g_.N, g_.C, g_.H, g_.W, device="cuda") * 7.0)
    dy.copy_(torch.randn(g_.N, g_.F, g_.OH, g_.OW, device="cuda"))
    g.replay()
    torch.cuda.synchronize()
    for o, exp in zip((y, dw, dx), want()):
        assert np.array_equal(_bits(o).reshape(-1), exp.reshape(-1))
