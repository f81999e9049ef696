"""The one-read slicing of long operands (launch_pslice) on the GPU.

An operand whose padded K is past the one-pass limit (column access: op(B) of an NN or TN GEMM,
op(A) of a TN or TT GEMM, past 3072; row access past 4096) is read once: blocks hold a 32-column
panel or an 8-row strip over a range of k in registers, and the blocks of a panel exchange their
partial maxima through slots in the workspace that the call marks empty first, through the
XCD's L2 (a column-access operand past K = 32768 takes parts 2.5 times as long, so that a
panel never has more than 26; past K = 66560 it takes the two passes). Checked against
the oracle: every digit of both operands' panels, the exponents, the zero padding and the
GEMM's bits, at S = 1..3, over every transpose, for K just past the limits, K with a partial
last part, ragged panels and long K; the same with the wait bound set to zero (every block then
reads its panel's whole K itself for the maxima, the fallback that keeps a block from depending
on another being resident or visible); on a workspace of constant bytes (the slots must be
marked by the call itself); and in strided batches.
"""
import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from bit_reproducible_training_amd import _lib
from gpu_util import bits, decode_digits, note, run, to_dev
from oracle import oracle as O

pytestmark = pytest.mark.gpu

# Padded K from just past the column one-pass limit (3072) to several parts of 1024 k, and past
# 32 such parts (K > 32768), where a column-access operand's parts are 2.5 times as long (2560 k:
# at most 26 parts, on one XCD), including the boundaries K = 32768 / 32769 and 66560 / 66561
# (26 wide parts / two passes for a column-access operand).
SHAPES = [(64, 100, 3076), (33, 200, 4096), (100, 33, 5000), (130, 70, 8193), (32, 32, 3073),
          (70, 45, 4097), (24, 40, 12289), (9, 17, 20000), (40, 33, 40000), (20, 64, 65536),
          (33, 40, 32768), (40, 20, 32769), (24, 40, 66560), (30, 20, 66561)]


def _check_slices(torch, A, B, M, N, K, ta, tb, S, ws_fill=None):
    cfg = rg.Config(slices=S, trans_a=ta, trans_b=tb, tile_m=64, tile_n=64)
    plan = rg.make_plan(M, N, K, cfg)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    if ws_fill is not None:
        ws.fill_(ws_fill)
    C, plan, ws = run(torch, A, B, M, N, K, cfg, ws=ws)
    X, Y, eA, eB = O.quantize(A, B, M, N, K, ta, tb, S)
    info = rg.workspace_layout(M, N, K, cfg)
    w = ws.cpu().numpy()
    for off, R, Xo, eo, eoff in ((info.qa, info.Mp, X, eA, info.ea),
                                 (info.qb, info.Np, Y, eB, info.eb)):
        d, Xg = decode_digits(w, off, R, info.Kp, S)
        assert np.abs(d[0]).max() <= 127
        if S > 1:
            assert d[1:].min() >= 0
        assert np.array_equal(Xg[:Xo.shape[0], :K], Xo)
        assert not Xg[Xo.shape[0]:].any() and not Xg[:, K:].any()
        e = w[eoff:eoff + 4 * R].view(np.int32)
        assert np.array_equal(e[:Xo.shape[0]], eo)
        assert not e[Xo.shape[0]:].any()
    assert np.array_equal(bits(C), O.cpu_gemm(A, B, M, N, K, ta, tb, S).view(np.uint32))


def _inputs(M, N, K, seed):
    rng = np.random.default_rng(seed)
    A = (rng.standard_normal(M * K) * 2.0 ** rng.integers(-20, 20, M * K)).astype(np.float32)
    B = rng.standard_normal(N * K).astype(np.float32)
    # a column's maximum in a late part only, a zero column, a huge value
    B[(K - 1) * N + 3 if N > 3 else 0] = 3e5
    A[:K] = 0.0
    return A, B


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("S", [1, 2, 3])
def test_one_read_slicing_against_oracle(torch_gpu, M, N, K, ta, tb, S):
    A, B = _inputs(M, N, K, M * 3 + N * 7 + K + 11 * ta + 5 * tb + S)
    note("pslice M=%d N=%d K=%d ta=%d tb=%d S=%d" % (M, N, K, ta, tb, S))
    _check_slices(torch_gpu, A, B, M, N, K, ta, tb, S)


@pytest.mark.parametrize("M,N,K,ta,tb", [(64, 100, 3076, 0, 0), (130, 70, 8193, 1, 0),
                                         (100, 33, 5000, 1, 1), (40, 70, 9000, 0, 1),
                                         (33, 20, 17000, 0, 0), (20, 40, 50000, 1, 0)])
def test_one_read_slicing_fallback(torch_gpu, M, N, K, ta, tb):
    """Wait bound 0: every block takes the fallback; same digits and bits."""
    A, B = _inputs(M, N, K, 99 + K)
    prev = _lib.lib.rg_test_set_spin_limit(0)
    try:
        note("pslice fallback M=%d N=%d K=%d ta=%d tb=%d" % (M, N, K, ta, tb))
        _check_slices(torch_gpu, A, B, M, N, K, ta, tb, 3)
    finally:
        _lib.lib.rg_test_set_spin_limit(prev)


@pytest.mark.parametrize("fill", [0xFF, 0x01])
def test_one_read_slicing_on_garbage_workspace(torch_gpu, fill):
    """The partial-maximum slots start from whatever the workspace holds (a constant fill can look
    like a published maximum): the call marks them empty itself before the one read, whether the
    other operand takes the one pass in the same launch or the one read too."""
    torch = torch_gpu
    for M, N, K, ta, tb in [(96, 64, 4100, 0, 0), (64, 96, 6000, 1, 0), (64, 96, 6000, 0, 1),
                            (32, 40, 40000, 0, 0)]:
        A, B = _inputs(M, N, K, fill + K)
        for rep in range(2):
            note("pslice garbage fill=%d M=%d N=%d K=%d ta=%d tb=%d rep %d" % (fill, M, N, K, ta, tb, rep))
            _check_slices(torch, A, B, M, N, K, ta, tb, 3, ws_fill=fill)


def test_one_read_slicing_repeated_calls_one_workspace(torch_gpu):
    """Back-to-back calls on one workspace, different inputs each time: the maxima a call leaves
    in the slots must never be taken for the next call's."""
    torch = torch_gpu
    M, N, K = 200, 160, 4500
    cfg = rg.Config(slices=3)
    plan = rg.make_plan(M, N, K, cfg)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    outs, wants = [], []
    for i in range(4):
        A, B = _inputs(M, N, K, 1000 + i)
        dA, dB = to_dev(torch, A), to_dev(torch, B)
        C = torch.empty((M, N), dtype=torch.float32, device="cuda")
        code = rg.repro_gemm_fp32_ws(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), M, N, K, cfg,
                                     ws.data_ptr(), ws.numel(),
                                     torch.cuda.current_stream().cuda_stream, None)
        assert code == 0
        outs.append((C, dA, dB))
        wants.append(O.cpu_gemm(A, B, M, N, K, 0, 0, 3).view(np.uint32))
    torch.cuda.synchronize()
    for (C, _, _), want in zip(outs, wants):
        assert np.array_equal(bits(C), want)


@pytest.mark.parametrize("ta,tb,K", [(0, 0, 4000), (1, 0, 4000), (0, 1, 6000), (1, 0, 40000),
                                     (0, 0, 36000)])
def test_one_read_slicing_batched(torch_gpu, ta, tb, K):
    torch = torch_gpu
    rng = np.random.default_rng(7 + ta + K)
    batch, M, N = 3, 45, 70
    a_shape = (batch, K, M) if ta else (batch, M, K)
    b_shape = (batch, N, K) if tb else (batch, K, N)
    A = (rng.standard_normal(a_shape) * 2.0 ** rng.integers(-20, 20, (batch, 1, 1))).astype(np.float32)
    B = rng.standard_normal(b_shape).astype(np.float32)
    note("pslice batched ta=%d tb=%d" % (ta, tb))
    C = rg.bmm(torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda(), ta, tb, 3)
    torch.cuda.synchronize()
    for i in range(batch):
        Mi, Ki = (A[i].shape[1], A[i].shape[0]) if ta else A[i].shape
        Ni = B[i].shape[0] if tb else B[i].shape[1]
        want = O.cpu_gemm(np.ascontiguousarray(A[i]), np.ascontiguousarray(B[i]), Mi, Ni, Ki, ta, tb, 3)
        assert np.array_equal(bits(C[i]), want.view(np.uint32)), i
