"""The one-launch kernel for small GEMMs (contract_small: slicing, MFMA contraction and rounding
of a 32x32 tile in one block) against the oracle, bit for bit.

The planner gives it plain GEMMs with K <= 512 and few tiles (the
LeNet layers of configuration 2); a pinned 32x32 tile forces it for any K <= 512. Covered: every
transpose at S = 1, 2, 3 on the configurations' shapes and on ragged ones (rows, columns and K
that are no multiple of 32, 16 or 4; one output), the hash tool's input distributions, the
stress pattern with results that overflow to infinity or round to -0.0, a grid of many tiles,
and equality with the pipeline's 64x64 and 128x128 tiles on the same inputs.
"""
import ctypes

import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from bit_reproducible_training_amd import _lib
from gpu_util import bits, note, run, to_dev
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SHAPES = [(256, 256, 256), (64, 120, 400), (64, 400, 120), (120, 400, 64), (64, 84, 120),
          (64, 120, 84), (84, 120, 64), (64, 10, 84), (64, 84, 10), (10, 84, 64),
          (1, 1, 1), (33, 47, 511), (31, 65, 17), (100, 3, 5), (7, 200, 512)]


def _operands(M, N, K, ta, tb, seed, dist):
    """Inputs drawn for op(A) [M][K] and op(B) [K][N], stored as the transposes ask."""
    A, B = O.gen_hash_inputs(M, N, K, seed, dist)
    As = np.ascontiguousarray(A.reshape(M, K).T) if ta else A
    Bs = np.ascontiguousarray(B.reshape(K, N).T) if tb else B
    return A, B, As.ravel(), Bs.ravel()


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_small_shapes_every_transpose_and_slice_count(torch_gpu, M, N, K):
    torch = torch_gpu
    for S in (1, 2, 3):
        for ta, tb in ((0, 0), (1, 0), (0, 1), (1, 1)):
            A, B, As, Bs = _operands(M, N, K, ta, tb, 100 * S + 2 * ta + tb, "normal")
            want = O.cpu_gemm(A, B, M, N, K, 0, 0, S).view(np.uint32)
            cfg = rg.Config(slices=S, trans_a=bool(ta), trans_b=bool(tb))
            note("small M=%d N=%d K=%d S=%d ta=%d tb=%d" % (M, N, K, S, ta, tb))
            C, plan, _ = run(torch, As, Bs, M, N, K, cfg)
            assert (plan.tile_m, plan.tile_n) == (32, 32)
            assert np.array_equal(bits(C), want), (M, N, K, S, ta, tb)


@pytest.mark.parametrize("dist", O.HASH_DISTS)
def test_small_hash_tool_distributions(torch_gpu, dist):
    torch = torch_gpu
    M, N, K = 96, 80, 384
    for S in (1, 2, 3):
        A, B = O.gen_hash_inputs(M, N, K, 777, dist)
        want = O.cpu_gemm(A, B, M, N, K, 0, 0, S).view(np.uint32)
        note("small dist=%s S=%d" % (dist, S))
        C, plan, _ = run(torch, A, B, M, N, K, rg.Config(slices=S))
        assert (plan.tile_m, plan.tile_n) == (32, 32)
        assert np.array_equal(bits(C), want), (dist, S)


def test_small_stress_overflow_and_negative_zero(torch_gpu):
    from test_oracle import _stress_inputs

    torch = torch_gpu
    rng = np.random.default_rng(19)
    M, N, K = 96, 60, 257
    A, B = _stress_inputs(M, N, K, rng)
    A[7] = np.float32(3e38)
    B[:, 5] = np.float32(2e38)     # row 7 x column 5 overflows
    A[11] = np.float32(-1e-45)
    B[:, 8] = np.float32(1e-45)    # tiny negative products round to -0.0
    for S in (1, 2, 3):
        want = O.cpu_gemm(A.ravel(), B.ravel(), M, N, K, 0, 0, S).view(np.uint32)
        note("small stress S=%d" % S)
        C, plan, _ = run(torch, A.ravel(), B.ravel(), M, N, K, rg.Config(slices=S))
        assert (plan.tile_m, plan.tile_n) == (32, 32)
        assert np.array_equal(bits(C), want), S


def test_small_pinned_tile_many_blocks_equals_pipeline(torch_gpu):
    """A pinned 32x32 tile on a shape with 1024 tiles gives the pipeline's bits (64x64 and
    128x128 tiles, split 1 and 3) and the oracle's."""
    torch = torch_gpu
    M, N, K = 1024, 1000, 500
    A = O.gen_normal(M * K, 1.0, 5)
    B = O.gen_normal(K * N, 1.0, 6)
    want = O.cpu_gemm(A, B, M, N, K, 0, 0, 3).view(np.uint32)
    dA, dB = to_dev(torch, A), to_dev(torch, B)
    for tm, tn, split in ((32, 32, 1), (64, 64, 1), (128, 128, 1), (64, 64, 3)):
        note("small vs pipeline tile %dx%d split %d" % (tm, tn, split))
        C, plan, _ = run(torch, dA, dB, M, N, K, rg.Config(tile_m=tm, tile_n=tn, split_k=split))
        assert (plan.tile_m, plan.tile_n) == (tm, tn)
        assert np.array_equal(bits(C), want), (tm, tn, split)


def test_small_noalloc_and_repeat(torch_gpu):
    """The allocation-free entry point takes the same kernel; repeated calls give the same bits."""
    torch = torch_gpu
    M, N, K = 64, 120, 400
    A = O.gen_normal(M * K, 1.0, 8)
    B = O.gen_normal(N * K, 1.0, 9)
    want = O.cpu_gemm(A, B, M, N, K, 0, 1, 3).view(np.uint32)
    dA, dB = to_dev(torch, A), to_dev(torch, B)
    cfg = rg.Config(trans_b=True)
    for rep in range(3):
        note("small repeat", rep)
        C, _, _ = run(torch, dA, dB, M, N, K, cfg)
        assert np.array_equal(bits(C), want), rep
    C = torch.full((M, N), float("nan"), device="cuda")
    note("small noalloc")
    c = cfg.to_c()
    code = _lib.lib.rg_gemm_fp32_noalloc(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), M, N, K,
                                         ctypes.byref(c), torch.cuda.current_stream().cuda_stream)
    assert code == 0, _lib.error_string(code)
    torch.cuda.synchronize()
    assert np.array_equal(bits(C), want)
