"""The reference's hash tool (repro_gemm_cuda/hash_repro_gemm.cu) restated on the GPU for all
its input distributions: uniform U[-1,1), normal, weights (N(0, 0.02) with 0.1% of the values
x100), wide (random sign x 2^U[-40,40]) and stress (zero, subnormal, 1e30 and signed-zero rows,
one 1e6 outlier; zero, 2^[-60,60] and 2^-120-scaled columns), inputs drawn as the tool draws them
(oracle.gen_hash_inputs).

As the tool does (hash_repro_gemm.cu:115-143), every algorithm x split_k in
{1, 2, 3, 4, 7, 8, 16, 64} x 2 runs must give one output hash, with C poisoned before each run;
unlike the tool, which checks the CPU definition only for one configuration, every run is compared
bit for bit with the oracle, at S = 1, 2 and 3.
"""
import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from gpu_util import bits, note, run, to_dev
from oracle import oracle as O

pytestmark = pytest.mark.gpu
ALGOS = [rg.Algo.Reference, rg.Algo.Tiled, rg.Algo.TensorCore, rg.Algo.Auto]
SPLITS = (1, 2, 3, 4, 7, 8, 16, 64)


@pytest.mark.parametrize("dist", O.HASH_DISTS)
@pytest.mark.parametrize("S", [1, 2, 3])
def test_hash_tool_distribution(torch_gpu, dist, S):
    torch = torch_gpu
    M, N, K = 256, 256, 1024                      # the tool's default shape
    A, B = O.gen_hash_inputs(M, N, K, 12345, dist)
    want = O.cpu_gemm(A, B, M, N, K, 0, 0, S).view(np.uint32)
    dA, dB = to_dev(torch, A), to_dev(torch, B)
    ws = None
    for algo in ALGOS:
        for split in SPLITS:
            for rep in range(2):
                note("hash dist=%s S=%d algo=%s split=%d run=%d" % (dist, S, algo.name, split, rep))
                C, _, ws = run(torch, dA, dB, M, N, K, rg.Config(algo=algo, slices=S, split_k=split), ws=ws)
                assert np.array_equal(bits(C), want), (dist, S, algo.name, split, rep)


@pytest.mark.parametrize("dist", ["uniform", "weights", "wide"])
def test_hash_tool_distributions_ragged_transposed(torch_gpu, dist):
    """The same distributions on a shape that is not a tile multiple, with every transpose."""
    torch = torch_gpu
    M, N, K = 133, 77, 301
    A, B = O.gen_hash_inputs(M, N, K, 4242, dist)
    At = np.ascontiguousarray(A.T)
    Bt = np.ascontiguousarray(B.T)
    for S in (1, 2, 3):
        want = O.cpu_gemm(A, B, M, N, K, 0, 0, S).view(np.uint32)
        for ta, tb in ((0, 0), (1, 0), (0, 1), (1, 1)):
            note("hash ragged dist=%s S=%d ta=%d tb=%d" % (dist, S, ta, tb))
            C, _, _ = run(torch, to_dev(torch, At if ta else A), to_dev(torch, Bt if tb else B), M, N, K,
                          rg.Config(slices=S, trans_a=bool(ta), trans_b=bool(tb)))
            assert np.array_equal(bits(C), want), (dist, S, ta, tb)
