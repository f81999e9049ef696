"""GEMM inputs holding NaN or infinities, on the CPU.

The definition is meant for finite inputs (the reference's hash tool refuses others,
hash_repro_gemm.cu:96-98), but the reference's CPU path still gives a result, and that result is
what every path here reproduces: the row and column maxima skip NaN (std::fmax,
repro_gemm_cpu.h:30-31, 36-37) and keep infinities, and fixed_point's (int)nearbyintf turns a
NaN or an infinity into INT_MIN on x86, clamped to -127 * 2^(7(S-1)) (repro_gemm_math.cuh:71-83).
The oracle is pinned against the reference's own CPU path compiled from its sources
(oracle/_ref, when built) and against two cases worked out by hand; the library's CPU path
(the compiled binding over include/repro_gemm_cpu.h) must give the same bits.
"""
import numpy as np
import pytest

from oracle import oracle as O


def nonfinite_inputs(M, N, K, seed):
    """N(0,1) operands with NaN and infinities planted in a few rows of A and columns of B:
    a lone +inf, a lone -inf, a lone NaN, a whole NaN row, NaN and +inf in one row, and in B a
    NaN and a -inf. A is M x K and B is N x K in memory; with transposes the same values land
    in other rows and columns, which the tests also run."""
    rng = np.random.default_rng(seed)
    A = rng.standard_normal(M * K).astype(np.float32)
    B = rng.standard_normal(N * K).astype(np.float32)
    A[3 * K + 5] = np.inf
    A[4 * K + 7] = -np.inf
    A[5 * K + 1] = np.nan
    A[6 * K:7 * K] = np.nan
    A[8 * K + 2] = np.nan
    A[8 * K + 9] = np.inf
    B[2 * K + 4] = np.nan
    B[11 * K + 3] = -np.inf
    return A, B


TRANSPOSES = [(0, 0), (1, 0), (0, 1), (1, 1)]


@pytest.mark.parametrize("S", [1, 2, 3])
def test_oracle_matches_reference_cpu_path_on_nonfinite_inputs(S):
    if O.ref is None:
        pytest.skip("oracle/_ref (the reference's CPU path) is not built here")
    M, N, K = 37, 29, 53
    A, B = nonfinite_inputs(M, N, K, 5)
    for ta, tb in TRANSPOSES:
        want = np.asarray(O.ref_cpu_gemm(A, B, M, N, K, ta, tb, S)).view(np.uint32).ravel()
        got = O.cpu_gemm(A, B, M, N, K, ta, tb, S).view(np.uint32).ravel()
        assert np.array_equal(got, want), (ta, tb)


def test_oracle_nonfinite_hand_cases():
    """Two GEMMs worked out by hand at S = 3 (lim = 127 * 2^14).
    A = [inf], B = [1]: e_A = scale_exponent(inf) = 128, X = -lim; e_B = -6 (1/127 <= 2^-6),
    Y = 2^20; T = -127 * 2^34 and E = 128 - 6 - 28 = 94, so C = -127 * 2^128 = -inf.
    A = [NaN, 2], B = [1, 0]: the maximum skips NaN, e_A = -5 (2/127 <= 2^-5), X = [-lim, 2^20];
    T = -127 * 2^34 and E = -5 - 6 - 28 = -39, so C = -127 / 32."""
    C = O.cpu_gemm(np.array([np.inf], np.float32), np.array([1.0], np.float32), 1, 1, 1, 0, 0, 3)
    assert np.isneginf(np.asarray(C).ravel()[0])
    C = O.cpu_gemm(np.array([np.nan, 2.0], np.float32), np.array([1.0, 0.0], np.float32), 1, 1, 2, 0, 0, 3)
    assert np.asarray(C).ravel()[0] == np.float32(-127.0 / 32.0)


@pytest.mark.parametrize("S", [1, 2, 3])
def test_cpu_path_matches_oracle_on_nonfinite_inputs(S):
    import torch

    import bit_reproducible_training_amd as rg

    for M, N, K in [(37, 29, 53), (70, 90, 1100)]:
        A, B = nonfinite_inputs(M, N, K, 6 + S)
        tA, tB = torch.from_numpy(A), torch.from_numpy(B)
        for ta, tb in TRANSPOSES:
            want = O.cpu_gemm(A, B, M, N, K, ta, tb, S).view(np.uint32).ravel()
            got = rg.gemm(tA, tB, M, N, K, ta=bool(ta), tb=bool(tb), S=S).numpy().view(np.uint32).ravel()
            assert np.array_equal(got, want), (M, N, K, ta, tb)
