"""The tensor operations on several streams at once.

Each call of rg.gemm / rg.exact_sum / rg.conv2d takes its workspace from PyTorch's caching
allocator on the current stream, so GEMMs queued on two streams that run at the same time never
share digit panels or partials. Here two streams each run a chain of different GEMMs, sums and
convolutions concurrently (no synchronisation between them until the end); every result must
equal the oracle bit for bit, and the inputs are freed and reallocated between rounds so the
allocator reuses memory across the two streams' lifetimes.
"""
import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from gpu_util import note
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().numpy().view(np.uint32)


def test_gemms_on_two_streams_match_the_oracle(torch_gpu):
    torch = torch_gpu
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]  # default priority
    shapes = [(512, 384, 1024, 0, 1), (256, 768, 512, 1, 0), (640, 320, 2048, 0, 0),
              (1024, 256, 768, 0, 1)]
    for rnd in range(3):
        jobs = []
        for si, stream in enumerate(streams):
            for j, (M, N, K, ta, tb) in enumerate(shapes):
                seed = 7000 + 100 * rnd + 10 * si + j
                A = O.gen_normal(M * K, 1.0, seed)
                B = O.gen_normal(K * N, 0.05, seed + 1)
                jobs.append((stream, M, N, K, ta, tb, A, B))
        outs = []
        note("two-stream round", rnd)
        for stream, M, N, K, ta, tb, A, B in jobs:
            with torch.cuda.stream(stream):
                dA = torch.from_numpy(A).to("cuda", non_blocking=False)
                dB = torch.from_numpy(B).to("cuda", non_blocking=False)
                C = rg.gemm(dA, dB, M, N, K, ta, tb, 3)
                s = rg.exact_sum(C, M, N, 1, False)
                outs.append((C, s))
                del dA, dB  # returned to the allocator while the stream may still run
        torch.cuda.synchronize()
        for (stream, M, N, K, ta, tb, A, B), (C, s) in zip(jobs, outs):
            want = O.cpu_gemm(A, B, M, N, K, ta, tb, 3)
            assert np.array_equal(_bits(C), want.view(np.uint32)), (rnd, M, N, K, ta, tb)
            assert np.array_equal(_bits(s), O.exact_sum(want, M, N, 1).view(np.uint32))


def test_convolutions_on_two_streams_match_the_oracle(torch_gpu):
    torch = torch_gpu
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    shape = (8, 6, 14, 14, 16, 5, 5, 1, 1, 0, 0)
    N, C, H, W, F, KH, KW, SY, SX, PY, PX = shape
    OH, OW = O.conv_out_hw(shape)
    jobs = []
    for si, stream in enumerate(streams):
        x = O.gen_normal(N * C * H * W, 1.0, 8100 + si)
        w = O.gen_normal(F * C * KH * KW, 0.1, 8110 + si)
        dy = O.gen_normal(N * F * OH * OW, 1e-3, 8120 + si)
        with torch.cuda.stream(stream):
            dx_ = torch.from_numpy(x).cuda().view(N, C, H, W)
            dw_ = torch.from_numpy(w).cuda().view(F, C, KH, KW)
            ddy = torch.from_numpy(dy).cuda().view(N, F, OH, OW)
            note("conv stream", si)
            res = (rg.conv2d(dx_, dw_, SY, SX, PY, PX, 3),
                   rg.conv2d_grad_weight(ddy, dx_, KH, KW, SY, SX, PY, PX, 3),
                   rg.conv2d_grad_input(ddy, dw_, [N, C, H, W], SY, SX, PY, PX, 3))
        jobs.append(((x, w, dy), res))
    torch.cuda.synchronize()
    for (x, w, dy), (y, gw, gx) in jobs:
        assert np.array_equal(_bits(y).ravel(), O.conv2d(x, w, shape).view(np.uint32).ravel())
        assert np.array_equal(_bits(gw).ravel(), O.conv2d_grad_weight(dy, x, shape).view(np.uint32).ravel())
        assert np.array_equal(_bits(gx).ravel(), O.conv2d_grad_input(dy, w, shape).view(np.uint32).ravel())


def test_gemm_out_argument_checks(torch_gpu):
    """out must be float32, on the inputs' device, contiguous, with M*N elements; a wrong one
    raises before any kernel is launched."""
    torch = torch_gpu
    A = torch.randn(8, 16, device="cuda")
    B = torch.randn(16, 4, device="cuda")
    good = torch.empty(8, 4, device="cuda")
    assert rg.gemm(A, B, 8, 4, 16, out=good) is good
    want = O.cpu_gemm(A.cpu().numpy(), B.cpu().numpy(), 8, 4, 16)
    assert np.array_equal(_bits(good), want.view(np.uint32))
    for bad in (torch.empty(8, 4, device="cuda", dtype=torch.float16), torch.empty(8, 3, device="cuda"),
                torch.empty(4, 8, device="cuda").t(), torch.empty(8, 4)):
        with pytest.raises(ValueError):
            rg.gemm(A, B, 8, 4, 16, out=bad)
    with pytest.raises(ValueError):
        rg.gemm(A, B.cpu(), 8, 4, 16)
    Ab = A.view(1, 8, 16)
    Bb = B.view(1, 16, 4)
    with pytest.raises(ValueError):
        rg.bmm(Ab, Bb, out=torch.empty(1, 8, 4, device="cuda", dtype=torch.float16))
    with pytest.raises(ValueError):
        rg.bmm(Ab, Bb, out=torch.empty(1, 8, 4))
